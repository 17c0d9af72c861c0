"""The min-p path's mass certificate against the reference's sequential mass.

k_full_pass (rust-llm_amd/csrc/full_kernels.h) finishes a min-p row only when
the top-p cut is the same for every mass in an interval [t_lo, t_hi] that it
proves holds the reference's target top_p * S_ref (sample.rs:307-324), where
S_ref is the f64 sequential sum of p_j = expf(fl(fl(l_j - M) / T)) in sorted
order. The interval and its constants are minp_bound.h's, built for the host
(tests/native/libminp_bound.so), so this checks the kernel's own bound.

The pass's arithmetic is emulated here step by step in the kernel's layout:
chunks of the row's float4s, steps of PASS_U float4 a thread (256 threads, four
waves), a wave's running maximum raised once per step with the partial sums
rescaled by 2^floor(z) exp2_hw(frac z), terms exp2_hw(fl(fl(l - m) c2)) summed
per lane in f32 (PASS_TERMS a step) and then in f64, the last chunk's
vocab % 4 elements, and the f64 combinations of waves and chunks. To stress
the bound, every f32 rounding of the pass goes one way (toward the larger
mass, or the smaller), and the hardware exp2 errs by its whole assumed bound
in that direction; the reference's side is computed as it is (round to
nearest, a correctly rounded expf). Rows: mass spread at |y| ~ ln V, near
|y| = K and beyond it, in the subnormal range, long rescale chains (a row
rising along each chunk, at the largest vocabulary and at 151 936), several
temperatures. A second test plants a mistake in the bound (only the
exponentials' own errors counted) and shows the emulation catches it.
"""
import ctypes
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "native", "libminp_bound.so")
F32 = np.float32
F64 = np.float64
LOG2E = 1.4426950408889634


def _lib():
    if not os.path.exists(LIB):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "native"), "libminp_bound.so"], check=True)
    L = ctypes.CDLL(LIB)
    L.minp_target_interval.argtypes = [ctypes.c_double, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float,
                                       ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
    L.minp_constants.argtypes = [ctypes.POINTER(ctypes.c_double)]
    return L


def constants():
    a = (ctypes.c_double * 10)()
    _lib().minp_constants(a)
    names = ["PASS_THREADS", "PASS_U", "PASS_TERMS", "HW_EXP2_REL", "MASS_K", "EPS_NEAR", "F32_STEP_REL",
             "MASS_REL", "RESCALE_REL", "MASS_ABS_PER_TERM"]
    return dict(zip(names, list(a)))


def interval(smid, V, C, top_p):
    lo, hi = ctypes.c_double(), ctypes.c_double()
    _lib().minp_target_interval(smid, V, C, top_p, ctypes.byref(lo), ctypes.byref(hi))
    return lo.value, hi.value


# ---------------------------------------------------- directed f32 rounding --
def _round_f32(x, err, d):
    """x + err (exact; err the f64 rounding error of x) rounded to f32:
    to nearest for d = 0, up for d = +1, down for d = -1."""
    r = x.astype(F32)
    if d == 0:
        return r
    r64 = r.astype(F64)
    if d > 0:
        bump = (r64 < x) | ((r64 == x) & (err > 0))
        return np.where(bump, np.nextafter(r, F32(np.inf)), r)
    bump = (r64 > x) | ((r64 == x) & (err < 0))
    return np.where(bump, np.nextafter(r, F32(-np.inf)), r)


def _two_sum(a, b):
    with np.errstate(invalid="ignore"):  # -inf operands (masked-out loads) give NaN errors, never used
        return _two_sum_raw(a, b)


def _two_sum_raw(a, b):
    s = a + b
    bb = s - a
    return s, (a - (s - bb)) + (b - bb)


def f32_add(a, b, d):
    s, e = _two_sum(a.astype(F64), b.astype(F64))
    return _round_f32(s, e, d)


def f32_mul(a, b, d):  # a product of two f32 is exact in f64
    return _round_f32(a.astype(F64) * b.astype(F64), np.zeros(np.shape(a), F64), d)


def exp2_hw(z, d, H):
    """The hardware exp2 of f32 z, erring by its whole assumed bound H
    toward d (the f32 rounding of the result included in H)."""
    t = np.exp2(z.astype(F64))
    if d == 0:
        return t.astype(F32)
    v = _round_f32(t * (1.0 + d * (H - 2.0 ** -23)), np.zeros_like(t), d)
    small = t < 2.0 ** -126  # flushed, or off by up to 2^-126 absolute
    return np.where(small, F32(2.0 ** -126) if d > 0 else F32(0.0), v)


def rescale(z, d, H):
    """2^z (z <= 0, f64) as the pass forms it: 2^floor(z) exactly times
    exp2_hw of the fraction rounded to f32."""
    z = np.asarray(z, F64)
    ok = z > -1100.0
    n = np.floor(np.where(ok, z, 0.0))
    frac = _round_f32(np.where(ok, z - n, 0.0), np.zeros_like(z), d)
    f = exp2_hw(frac, d, H).astype(F64)
    return np.where(ok, np.ldexp(f, n.astype(np.int64)), 0.0)


# ------------------------------------------------------ the pass, emulated --
def pass_mass(row, T, C, d, K):
    """k_full_pass's mass for one row (penalty already applied), relative to
    the row's maximum, with every f32 rounding toward d."""
    V = row.size
    nt, U = int(K["PASS_THREADS"]), int(K["PASS_U"])
    step = nt * U
    H = K["HW_EXP2_REL"]
    invT = 1.0 / float(F64(F32(T)))
    log2e_T = LOG2E * invT
    c2 = _round_f32(np.array([log2e_T]), np.zeros(1), -d)[0]  # a larger c2 gives a smaller mass
    n4 = V // 4
    v4 = row[: 4 * n4].reshape(n4, 4)
    tid = np.arange(nt)
    wave_of = tid // 64
    Mc_all, Sc_all = [], []
    for c in range(C):
        q0, q1 = n4 * c // C, n4 * (c + 1) // C
        m_run = np.full(4, -np.inf, F32)
        S = np.zeros(nt, F64)
        for b in range(q0, q1, step):
            qq = b + np.arange(U)[None, :] * nt + tid[:, None]           # [tid, u]
            ok = qq < q1
            A = np.where(ok[..., None], v4[np.minimum(qq, q1 - 1)], F32(-np.inf))  # [tid, u, 4]
            tmax = A.reshape(4, 64 * U * 4).max(axis=1)
            rise = tmax > m_run
            was = m_run > -np.inf
            fac = np.ones(4, F64)
            sel = rise & was
            if sel.any():
                fac[sel] = rescale((m_run[sel].astype(F64) - tmax[sel].astype(F64)) * log2e_T, d, H)
            S = S * fac[wave_of]
            m_run = np.where(rise, tmax, m_run)
            diff = f32_add(A, -np.broadcast_to(m_run[wave_of][:, None, None], A.shape).astype(F32), d)
            z = f32_mul(diff, np.full(A.shape, c2, F32), d)
            q = exp2_hw(z, d, H)
            acc = np.zeros(nt, F32)
            for u in range(U):
                for k in range(4):
                    acc = np.where(ok[:, u], f32_add(acc, q[:, u, k], d), acc)
            S = S + acc.astype(F64)
        if c == C - 1 and V > 4 * n4:
            # The last vocab % 4 elements, lane e - 4 n4 of wave 0: one wave
            # maximum over them, an f64 rescaling, then their terms.
            tail = row[4 * n4:]
            x = tail.max()
            if x > m_run[0]:
                if m_run[0] > -np.inf:
                    S[wave_of == 0] *= math.exp((float(m_run[0]) - float(x)) * invT)
                m_run[0] = x
            diff = f32_add(tail, np.full(tail.shape, -m_run[0], F32), d)
            z = f32_mul(diff, np.full(tail.shape, c2, F32), d)
            S[: tail.size] += exp2_hw(z, d, H).astype(F64)
        Sw = np.array([S[wave_of == w].sum() for w in range(4)])
        Mc = m_run.max()
        Sc = sum(Sw[w] * math.exp((float(m_run[w]) - float(Mc)) * invT) for w in range(4) if m_run[w] > -np.inf)
        Mc_all.append(Mc)
        Sc_all.append(Sc)
    M = max(Mc_all)
    return sum(s * math.exp((float(m) - float(M)) * invT) for m, s in zip(Mc_all, Sc_all))


def reference_target(row, T, top_p):
    """top_p * S_ref as the reference computes it (sample.rs:307-324)."""
    M = row.max()
    x = (row - M).astype(F32) / F32(T)
    p = np.exp(x.astype(F64)).astype(F32)  # correctly rounded expf
    s = np.add.accumulate(np.sort(p)[::-1].astype(F64))[-1]
    return float(F64(F32(top_p)) * s)


# -------------------------------------------------------------- the rows --
def rows_for_the_bound():
    rng = np.random.default_rng(2025)
    out = []
    V1, VMAX = 151936, 1 << 21
    lnV = math.log(V1)
    # Mass spread at |y| ~ ln V: one maximum, the rest about ln V below it.
    r = np.full(V1, -lnV, F32) + rng.normal(0, 0.3, V1).astype(F32)
    r[rng.integers(V1)] = 0.0
    out.append(("mass at ln V", r, 1.0, 16))
    out.append(("mass at ln V, T 0.7", (r * F32(0.7)).astype(F32), 0.7, 16))
    # A ragged vocabulary whose maximum is among the last vocab % 4 elements.
    Vr = 100003
    r = np.full(Vr, -math.log(Vr), F32) + rng.normal(0, 0.3, Vr).astype(F32)
    r[Vr - 2] = 0.0
    out.append(("ragged, maximum in the tail", r, 1.0, 24))
    # Mass near |y| = K = 32 and just beyond, and in the subnormal range.
    r = np.where(rng.random(V1) < 0.5, F32(-31.9), F32(-32.1)).astype(F32)
    r[7] = 0.0
    out.append(("terms at K", r, 1.0, 16))
    r = rng.uniform(-104.0, -87.0, V1).astype(F32)
    r[11] = 0.0
    out.append(("subnormal terms", r, 1.0, 16))
    # Nearly flat rows: every |y| small, a mass of about V.
    r = rng.normal(0, 0.01, V1).astype(F32)
    out.append(("flat", r, 1.0, 16))
    out.append(("flat, T 4", r, 4.0, 16))
    out.append(("flat, T 0.05", r, 0.05, 16))
    # The zipf workload's shape: N(0, 3^2) plus -1.1 ln(rank) over a permuted order.
    r = (rng.normal(0, 3.0, V1) - 1.1 * np.log(1 + rng.permutation(V1))).astype(F32)
    out.append(("zipf", r, 1.0, 16))
    # Long rescale chains: each chunk rises along its float4s, so every step
    # raises every wave's maximum (V = 2^21: 32 chunks of seven steps; V1:
    # four chunks of four steps).
    for V, C in ((VMAX, 32), (V1, 4)):
        ramp = np.linspace(-12.0, 0.0, V).astype(F32)
        r = (ramp + rng.normal(0, 0.05, V).astype(F32)).astype(F32)
        out.append(("rising, V %d, %d chunks" % (V, C), r, 1.0, C))
        out.append(("rising, V %d, %d chunks, T 0.6" % (V, C), r, 0.6, C))
    return out


ROWS = rows_for_the_bound()


@pytest.mark.parametrize("name,row,T,C", ROWS, ids=[r[0] for r in ROWS])
def test_the_interval_holds_the_reference_target(name, row, T, C):
    K = constants()
    top_p = 0.95
    want = reference_target(row, T, top_p)
    for d in (1, -1, 0):
        smid = pass_mass(row, T, C, d, K)
        lo, hi = interval(smid, row.size, C, top_p)
        print("%s d=%+d: target %.17g in [%.17g, %.17g], slack below %.3g, above %.3g (relative)"
              % (name, d, want, lo, hi, (want - lo) / want, (hi - want) / want))
        assert lo <= want <= hi, (name, d, lo, want, hi)


def test_the_f32_step_term_covers_the_loop():
    # The pass adds PASS_TERMS = 4 * PASS_U terms per lane per step in f32:
    # PASS_TERMS - 1 roundings, gamma_(PASS_TERMS - 1).
    K = constants()
    assert K["PASS_TERMS"] == 4 * K["PASS_U"]
    n = K["PASS_TERMS"] - 1
    u = 2.0 ** -24
    assert K["F32_STEP_REL"] >= n * u / (1 - n * u)
    assert K["MASS_REL"] >= K["EPS_NEAR"] / (1 - K["EPS_NEAR"]) + K["F32_STEP_REL"]


def test_a_bound_from_the_exponentials_alone_fails_on_mass_at_ln_v():
    # Planted in the bound, not in the pass: an interval that counts only the
    # exponentials' own errors (libm's 0.502 ulp and the hardware exp2's H),
    # leaving out the roundings of the argument (which grow with |y|), the f32
    # step sums and the rescalings. On the mass-at-ln-V row, with the pass's
    # roundings toward the larger mass, the reference's target falls outside
    # it: the emulation resolves errors of that size, so the shipped bound's
    # extra terms are needed, not decoration.
    K = constants()
    name, row, T, C = ROWS[0]
    top_p = 0.95
    want = reference_target(row, T, top_p)
    smid = pass_mass(row, T, C, 1, K)
    V = row.size
    rel = (1.004 * 2.0 ** -24 + K["HW_EXP2_REL"]) * (1 + 2.0 ** -7)
    s_lo = (smid * (1 - rel) - K["MASS_ABS_PER_TERM"] * V) * (1 - (V + 64) * 2.0 ** -53)
    s_hi = (smid * (1 + rel) + K["MASS_ABS_PER_TERM"] * V) * (1 + (V + 64) * 2.0 ** -53)
    lo, hi = top_p * s_lo * (1 - 2.0 ** -48), top_p * s_hi * (1 + 2.0 ** -48)
    print("naive bound: [%.17g, %.17g], target %.17g" % (lo, hi, want))
    assert not (lo <= want <= hi), (lo, want, hi)
    # and the shipped interval holds it
    lo, hi = interval(smid, V, C, top_p)
    assert lo <= want <= hi
