"""Python bindings (ctypes) for librl_sampler.so, the gfx950 token sampler and
output head.

The library's C ABI is include/rl_sampler.h (device batch entry points),
include/rl_sampler_host.h (the reference's Sampler API kept on the host) and
include/rl_head.h (the Q6_K output head that writes logits into HBM). This
module only marshals arguments: every pick runs in the HIP library, and loading
fails loudly when the library has not been built.

Device buffers are torch tensors on a ROCm device (torch is used for device
memory and streams only).
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librl_sampler.so")

RL_OK = 0
RL_ERR_ARGUMENT = 1
RL_ERR_VOCAB = 2
RL_ERR_CAPACITY = 3
RL_ERR_DEVICE = 4
RL_ERR_NOT_CONFIGURED = 5


class Sampling(ctypes.Structure):
    """rl_sampling: the repr(C) mirror of Sampling (sample.rs:50-67)."""

    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repeat_penalty", ctypes.c_float),
        ("top_k", ctypes.c_uint64),
        ("repeat_last_n", ctypes.c_uint64),
        ("seed", ctypes.c_uint64),
    ]

    def __repr__(self):
        return ("Sampling(temperature=%r, top_k=%d, top_p=%r, min_p=%r, repeat_penalty=%r, "
                "repeat_last_n=%d, seed=%d)" % (self.temperature, self.top_k, self.top_p, self.min_p,
                                                self.repeat_penalty, self.repeat_last_n, self.seed))


class Rng(ctypes.Structure):
    _fields_ = [("s", ctypes.c_uint64 * 4)]


def sampling(temperature=0.6, top_k=20, top_p=0.95, min_p=0.0, repeat_penalty=1.0, repeat_last_n=64, seed=0):
    """Sampling::default() (sample.rs:88-100) unless overridden."""
    return Sampling(temperature, top_p, min_p, repeat_penalty, top_k, repeat_last_n, seed)


def greedy_sampling(**kw):
    """Sampling::GREEDY (sample.rs:71-79) unless overridden."""
    d = dict(temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=1.0, repeat_last_n=0, seed=0)
    d.update(kw)
    return sampling(**d)


class SamplerError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("rl_sampler error %d: %s" % (code, msg))
        self.code = code


_lib = None
_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64


def lib():
    """Loads the HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("%s is missing: build it with `make -C rust-llm_amd` "
                               "(or __graft_entry__.build())" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        L.rl_sampler_create.argtypes = [ctypes.c_int, _u32, _u32, _u32, ctypes.POINTER(_vp)]
        L.rl_sampler_destroy.argtypes = [_vp]
        L.rl_sampler_destroy.restype = None
        L.rl_sampler_configure.argtypes = [_vp, ctypes.POINTER(Sampling), _u32]
        L.rl_sampler_required_cand_stride.argtypes = [_vp, ctypes.POINTER(_u64)]
        L.rl_sampler_sample_rows.argtypes = [
            _vp, _vp, _u64, _u32, _u32, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u64, _vp]
        L.rl_argmax_rows.argtypes = [_vp, _vp, _u64, _u32, _u32, _vp, _vp]
        L.rl_argmax_rows_noalloc.argtypes = [ctypes.c_int, _vp, _u64, _u32, _u32, _vp, _vp]
        L.rl_top_probability_rows.argtypes = [_vp, _vp, _u64, _u32, _u32, _vp, _vp, _vp]
        L.rl_sampler_last_error.restype = ctypes.c_char_p
        L.rl_sampler_expf_range.argtypes = [_u32, _u64, _vp, _vp]
        L.rl_rng_seeded.argtypes = [ctypes.POINTER(Rng), _u64]
        L.rl_rng_seeded.restype = None
        L.rl_rng_next_u64.argtypes = [ctypes.POINTER(Rng)]
        L.rl_rng_next_u64.restype = _u64
        L.rl_rng_next_f32.argtypes = [ctypes.POINTER(Rng)]
        L.rl_rng_next_f32.restype = ctypes.c_float
        L.rl_sampling_default.restype = Sampling
        L.rl_sampling_greedy.restype = Sampling
        L.rl_entropy_seed.restype = _u64
        L.rl_host_argmax.argtypes = [ctypes.c_int, _vp, ctypes.c_size_t, ctypes.POINTER(_u32)]
        L.rl_host_sampler_new.argtypes = [ctypes.c_int, ctypes.c_size_t, ctypes.POINTER(Sampling), _u32,
                                          ctypes.POINTER(_vp)]
        L.rl_host_sampler_free.argtypes = [_vp]
        L.rl_host_sampler_free.restype = None
        L.rl_host_sampler_settings.argtypes = [_vp]
        L.rl_host_sampler_settings.restype = Sampling
        L.rl_host_sampler_reset.argtypes = [_vp]
        L.rl_host_sampler_reset.restype = None
        L.rl_host_sampler_remember.argtypes = [_vp, _u32]
        L.rl_host_sampler_remember.restype = None
        L.rl_host_sampler_sample.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.POINTER(_u32)]
        L.rl_host_sampler_sample_device.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.POINTER(_u32), _vp]
        L.rl_host_sampler_candidates.argtypes = [_vp, ctypes.POINTER(ctypes.POINTER(_u32)),
                                                 ctypes.POINTER(ctypes.POINTER(ctypes.c_float))]
        L.rl_host_sampler_candidates.restype = ctypes.c_size_t
        L.rl_host_sampler_rng.argtypes = [_vp, ctypes.POINTER(Rng)]
        L.rl_host_sampler_rng.restype = None
        L.rl_host_sampler_verify.argtypes = [_vp, _vp, _u64, ctypes.c_size_t, _vp, _u32, _vp, _vp]
        L.rl_host_sampler_commit_verified.argtypes = [_vp, _u32, ctypes.POINTER(_u32)]
        L.rl_host_sample_batch.argtypes = [ctypes.POINTER(_vp), _u32, _vp, _u64, ctypes.c_size_t, _vp, _vp]
        L.rl_head_create.argtypes = [ctypes.c_int, _u32, _u32, _u32, _vp, _u64, ctypes.POINTER(_vp)]
        L.rl_head_destroy.argtypes = [_vp]
        L.rl_head_destroy.restype = None
        L.rl_head_logits.argtypes = [_vp, _vp, _u32, _vp, _u64, _vp]
        L.rl_head_embed_rows.argtypes = [_vp, _vp, _u32, _vp, _u64, _vp]
        L.rl_quantize_rows.argtypes = [_vp, _u32, _u32, _vp, _vp, _vp, _vp]
        _lib = L
    return _lib


def _check(rc):
    if rc != RL_OK:
        raise SamplerError(rc, lib().rl_sampler_last_error().decode(errors="replace"))


def _ptr(t):
    """Device (or host numpy) buffer address, or None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def current_stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


class RngStream:
    """The reference's Rng (sample.rs:368-404), as the library implements it."""

    def __init__(self, seed):
        self.r = Rng()
        lib().rl_rng_seeded(ctypes.byref(self.r), seed)

    def next_u64(self):
        return lib().rl_rng_next_u64(ctypes.byref(self.r))

    def next_f32(self):
        return lib().rl_rng_next_f32(ctypes.byref(self.r))

    def state(self):
        return tuple(self.r.s)


class DeviceSampler:
    """A device context: rl_sampler_create / configure / sample_rows."""

    def __init__(self, max_rows, vocab, max_window=64, device=0):
        h = _vp()
        _check(lib().rl_sampler_create(device, max_rows, vocab, max_window, ctypes.byref(h)))
        self.h = h
        self.vocab = vocab
        self.max_rows = max_rows
        self.max_window = max_window

    def close(self):
        if getattr(self, "h", None):
            lib().rl_sampler_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def configure(self, settings):
        if isinstance(settings, Sampling):
            settings = [settings]
        arr = (Sampling * len(settings))(*settings)
        _check(lib().rl_sampler_configure(self.h, arr, len(settings)))

    def required_cand_stride(self):
        out = _u64()
        _check(lib().rl_sampler_required_cand_stride(self.h, ctypes.byref(out)))
        return out.value

    def sample_rows(self, logits, rows, row_stride, out_token, out_kept, out_used, windows=None,
                    window_stride=0, window_len=None, uniforms=None, out_ids=None, out_probs=None,
                    cand_stride=0, vocab=None, stream=None):
        _check(lib().rl_sampler_sample_rows(
            self.h, _ptr(logits), row_stride, rows, self.vocab if vocab is None else vocab,
            _ptr(windows), window_stride, _ptr(window_len), _ptr(uniforms),
            _ptr(out_token), _ptr(out_kept), _ptr(out_used), _ptr(out_ids), _ptr(out_probs), cand_stride,
            current_stream() if stream is None else stream))

    def argmax_rows(self, logits, rows, row_stride, out_token, vocab=None, stream=None):
        _check(lib().rl_argmax_rows(self.h, _ptr(logits), row_stride, rows,
                                    self.vocab if vocab is None else vocab, _ptr(out_token),
                                    current_stream() if stream is None else stream))


    def top_probability_rows(self, logits, rows, row_stride, out_token, out_prob, vocab=None, stream=None):
        """rl_top_probability_rows: argmax and 1 / sum exp(l - l_best) per row
        (forward.rs:1671-1680)."""
        _check(lib().rl_top_probability_rows(self.h, _ptr(logits), row_stride, rows,
                                             self.vocab if vocab is None else vocab, _ptr(out_token),
                                             _ptr(out_prob), current_stream() if stream is None else stream))


class BatchResult:
    def __init__(self, token, kept, used, ids, probs):
        self.token, self.kept, self.used, self.ids, self.probs = token, kept, used, ids, probs

    def candidates(self, r):
        k = int(self.kept[r])
        return self.ids[r, :k], self.probs[r, :k]


def sample_batch(ctx, logits, settings, windows=None, window_len=None, uniforms=None, with_candidates=True,
                 stream=None):
    """Configures `ctx` with `settings` (one per row), samples every row of the
    2-D device tensor `logits`, and returns host numpy results."""
    import torch
    rows, vocab = logits.shape
    dev = logits.device
    ctx.configure(settings)
    cs = ctx.required_cand_stride() if with_candidates else 0
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    kept = torch.empty(rows, dtype=torch.int32, device=dev)
    used = torch.empty(rows, dtype=torch.uint8, device=dev)
    ids = torch.empty((rows, cs), dtype=torch.int32, device=dev) if with_candidates else None
    probs = torch.empty((rows, cs), dtype=torch.float32, device=dev) if with_candidates else None
    ws = 0
    if windows is not None:
        ws = windows.shape[1]
    ctx.sample_rows(logits, rows, logits.stride(0), tok, kept, used, windows=windows, window_stride=ws,
                    window_len=window_len, uniforms=uniforms, out_ids=ids, out_probs=probs, cand_stride=cs,
                    vocab=vocab, stream=stream)
    torch.cuda.synchronize(dev)
    return BatchResult(tok.cpu().numpy().view("uint32"), kept.cpu().numpy().view("uint32"), used.cpu().numpy(),
                       ids.cpu().numpy().view("uint32") if ids is not None else None,
                       probs.cpu().numpy() if probs is not None else None)


class HostSampler:
    """The reference's Sampler API (sample.rs:132-219) over the host mirror."""

    def __init__(self, vocab, settings, max_rows=1, device=0):
        h = _vp()
        _check(lib().rl_host_sampler_new(device, vocab, ctypes.byref(settings), max_rows, ctypes.byref(h)))
        self.h = h
        self.vocab = vocab

    @classmethod
    def greedy(cls, vocab, device=0):
        return cls(vocab, lib().rl_sampling_greedy(), device=device)

    def close(self):
        if getattr(self, "h", None):
            lib().rl_host_sampler_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def settings(self):
        return lib().rl_host_sampler_settings(self.h)

    def reset(self):
        lib().rl_host_sampler_reset(self.h)

    def remember(self, token):
        lib().rl_host_sampler_remember(self.h, token)

    def sample(self, logits):
        """logits: host numpy float32 (copied to the GPU) or a 1-D device tensor."""
        out = _u32()
        if hasattr(logits, "data_ptr"):
            _check(lib().rl_host_sampler_sample_device(self.h, logits.data_ptr(), logits.numel(),
                                                       ctypes.byref(out), current_stream()))
        else:
            import numpy as np
            a = np.ascontiguousarray(logits, dtype=np.float32)
            _check(lib().rl_host_sampler_sample(self.h, a.ctypes.data, a.size, ctypes.byref(out)))
        return out.value

    def candidates(self):
        import numpy as np
        ip = ctypes.POINTER(_u32)()
        pp = ctypes.POINTER(ctypes.c_float)()
        n = lib().rl_host_sampler_candidates(self.h, ctypes.byref(ip), ctypes.byref(pp))
        if n == 0:
            return np.zeros(0, np.uint32), np.zeros(0, np.float32)
        return (np.ctypeslib.as_array(ip, shape=(n,)).copy(), np.ctypeslib.as_array(pp, shape=(n,)).copy())

    def rng_state(self):
        r = Rng()
        lib().rl_host_sampler_rng(self.h, ctypes.byref(r))
        return tuple(r.s)

    def verify(self, rows, drafts):
        """rows: 2-D device tensor of len(drafts)+1 logit rows. Returns the
        picks (uncommitted)."""
        import numpy as np
        d = np.ascontiguousarray(drafts, dtype=np.uint32)
        picks = np.zeros(d.size + 1, np.uint32)
        _check(lib().rl_host_sampler_verify(self.h, rows.data_ptr(), rows.stride(0), rows.shape[1],
                                            d.ctypes.data if d.size else None, d.size, picks.ctypes.data,
                                            current_stream()))
        return picks

    def commit_verified(self, row):
        """Commits verify row `row`; returns the committed token."""
        out = _u32()
        _check(lib().rl_host_sampler_commit_verified(self.h, row, ctypes.byref(out)))
        return out.value


def host_sample_batch(samplers, logits):
    """One device call over many samplers; logits is a 2-D device tensor."""
    import numpy as np
    n = len(samplers)
    arr = (_vp * n)(*[s.h for s in samplers])
    out = np.zeros(n, np.uint32)
    _check(lib().rl_host_sample_batch(arr, n, logits.data_ptr(), logits.stride(0), logits.shape[1],
                                      out.ctypes.data, current_stream()))
    return out


def argmax_rows_noalloc(logits, rows, row_stride, out_token, vocab, device=0, stream=None):
    """rl_argmax_rows_noalloc: per-row argmax (sample.rs:118-128) with no
    context and no allocation (its scratch is a fixed device array)."""
    _check(lib().rl_argmax_rows_noalloc(device, _ptr(logits), row_stride, rows, vocab, _ptr(out_token),
                                        current_stream() if stream is None else stream))


def host_argmax(logits, device=0):
    import numpy as np
    a = np.ascontiguousarray(logits, dtype=np.float32)
    out = _u32()
    _check(lib().rl_host_argmax(device, a.ctypes.data, a.size, ctypes.byref(out)))
    return out.value


def expf_range(lo_bits, out, stream=None):
    """Fills the device tensor `out` with the device expf of bit patterns
    lo_bits, lo_bits+1, ..."""
    _check(lib().rl_sampler_expf_range(lo_bits, out.numel(), out.data_ptr(),
                                       current_stream() if stream is None else stream))


def entropy_seed():
    return lib().rl_entropy_seed()


QK = 256
Q6K_BYTES = 210


class DeviceHead:
    """rl_head_create / rl_head_logits: the tied Q6_K output head
    (forward.rs:932-937) with its weights resident in HBM."""

    def __init__(self, q6k, k, rows, max_batch=32, device=0):
        import numpy as np
        w = np.ascontiguousarray(q6k, dtype=np.uint8)
        h = _vp()
        _check(lib().rl_head_create(device, k, rows, max_batch, w.ctypes.data, w.nbytes, ctypes.byref(h)))
        self.h = h
        self.k, self.rows, self.max_batch, self.device = k, rows, max_batch, device

    def close(self):
        if getattr(self, "h", None):
            lib().rl_head_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def logits_into(self, x, out, row_stride=None, stream=None):
        """x: device f32 [t][k] (contiguous); out: device f32 with rows of
        row_stride >= vocabulary entries."""
        t = x.shape[0]
        _check(lib().rl_head_logits(self.h, _ptr(x), t, _ptr(out),
                                    self.rows if row_stride is None else row_stride,
                                    current_stream() if stream is None else stream))

    def logits(self, x):
        import torch
        assert x.dtype == torch.float32 and x.is_contiguous() and x.shape[1] == self.k
        out = torch.empty((x.shape[0], self.rows), dtype=torch.float32, device=x.device)
        self.logits_into(x, out)
        return out

    def embed_into(self, tokens, out, row_stride=None, stream=None):
        """rl_head_embed_rows (forward.rs:1127-1138): tokens device int32/uint32
        [t]; out device f32 with rows of row_stride >= k entries."""
        t = tokens.shape[0]
        _check(lib().rl_head_embed_rows(self.h, _ptr(tokens), t, _ptr(out),
                                        self.k if row_stride is None else row_stride,
                                        current_stream() if stream is None else stream))

    def embed(self, tokens):
        """The embedding rows of device tokens [t] (int32 holding u32 ids), as a
        device f32 [t][k] tensor."""
        import torch
        assert tokens.dtype == torch.int32 and tokens.is_contiguous() and tokens.dim() == 1
        out = torch.empty((tokens.shape[0], self.k), dtype=torch.float32, device=tokens.device)
        self.embed_into(tokens, out)
        return out


def quantize_rows(x, stream=None):
    """rl_quantize_rows (quant.rs:337-375) of a device f32 [t][k] tensor:
    (d [t][nb], qs [t][nb*256] int8, bsums [t][nb][16] int16), device tensors."""
    import torch
    assert x.dtype == torch.float32 and x.is_contiguous()
    t, k = x.shape
    nb = -(-k // QK)
    d = torch.empty((t, nb), dtype=torch.float32, device=x.device)
    qs = torch.empty((t, nb * QK), dtype=torch.int8, device=x.device)
    bs = torch.empty((t, nb, 16), dtype=torch.int16, device=x.device)
    _check(lib().rl_quantize_rows(_ptr(x), t, k, _ptr(d), _ptr(qs), _ptr(bs),
                                  current_stream() if stream is None else stream))
    return d, qs, bs
