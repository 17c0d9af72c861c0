// The output head on gfx950: logits = token_embd (Q6_K, [k, rows]) times the
// normed hidden rows, bit-identical to rust-llm's CPU head
// (crates/rust-llm/src/forward.rs:932-937 → forward.rs:1157-1180 →
// crates/rust-llm/src/pool.rs:468-506 → crates/llm-core/src/kernels/mod.rs:273-300).
//
// What the bits depend on. The reference quantizes each activation row in
// blocks of 256 to int8 with one f32 scale per block (quant.rs:337-375), then
// per (token, vocabulary row) sums, block by block from 0.0 in f32,
//     (act.d * w.d) * (float)isum,   isum = sum_i s_{i/16} * (q_i - 32) * a_i,
// where isum is an exact i32. Any order of the integer work gives the same
// isum; the f32 line is kept as is, one lane per vocabulary row. So the device
// result equals the reference's whatever the tiling, with no tolerance.
//
// Layouts in HBM (built once by k_q6k_repack from the GGUF bytes):
//   wq  uint4 [groups][nb][13][64]: lane l of group g is vocabulary row
//       g*64 + l. Per lane and block, 13 16-byte chunks: chunks 3p, 3p+1, 3p+2
//       hold sub-blocks 4p..4p+3 as {L0,L1} pairs and their H words (below),
//       chunk 12 holds the 16 signed sub-block scales. A wave's load of one
//       chunk is 1 KiB contiguous.
//   wd  u16 [groups][nb][64]: the block's f16 scale.
//   Per sub-block of 16 unsigned 6-bit quants w_0..w_15 (ggml's value before
//   the -32): L0 byte b = w_b & 15 | (w_{4+b} & 15) << 4, L1 byte b =
//   w_{8+b} & 15 | (w_{12+b} & 15) << 4, H byte b = the high two bits of w_b,
//   w_{4+b}, w_{8+b}, w_{12+b} at bits 0, 2, 4, 6. Unpacking gives the four
//   dwords of bytes w_{4g..4g+3}, matching activation dword g of the sub-block.
//   Total bytes equal the GGUF tensor's (208 + 2 per block and row).
//   act u32 [t][nb][84]: per activation block, 64 dwords of int8 quants, 16
//       words c_j = -32 * bsum_j (the constant -32 folded into the starting
//       value of each sub-block's dot), the f32 scale, 3 words of padding.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rl {

constexpr int QK = 256;             // values per quantization block (quant.rs:12)
constexpr int Q6K_BLOCK_BYTES = 210; // ql 128, qh 64, scales 16, d f16 (quant.rs:19)
constexpr int HEAD_LANES = 64;       // vocabulary rows per group (one wave)
constexpr int HEAD_CHUNKS = 13;      // 16-byte chunks per lane and block
constexpr int ACT_WORDS = 84;        // u32 per activation block in the head's layout
constexpr int HEAD_WAVES = 4;        // waves (groups) per workgroup
constexpr int HEAD_THREADS = HEAD_WAVES * HEAD_LANES;
constexpr int HEAD_TMAX = 32;        // activation rows one pass takes

// ---------------------------------------------------------------- repack

// The unsigned 6-bit quant at activation index i of a ggml Q6_K block
// (kernels/mod.rs:281-296: index h*128 + g*32 + l reads ql_h[l] or
// ql_h[32 + l], low or high nibble by g, and bits 2g..2g+1 of qh_h[l]).
__device__ inline uint32_t q6k_quant_at(const uint8_t *b, int i) {
    const int h = i >> 7, g = (i >> 5) & 3, l = i & 31;
    const uint8_t lo = b[h * 64 + (g & 1) * 32 + l];
    const uint32_t low = (g & 2) ? (lo >> 4) : (lo & 15);
    const uint32_t high = (b[128 + h * 32 + l] >> (2 * g)) & 3;
    return low | (high << 4);
}

// One thread per (group, block, lane); lanes are innermost so the 16-byte
// stores of a wave are contiguous. Rows at or past `rows` are zero.
__global__ void k_q6k_repack(const uint8_t *__restrict__ src, uint32_t rows, uint32_t nb, uint32_t groups,
                             uint4 *__restrict__ wq, uint16_t *__restrict__ wd) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t total = (uint64_t)groups * nb * HEAD_LANES;
    if (idx >= total) return;
    const uint32_t lane = (uint32_t)(idx % HEAD_LANES);
    const uint64_t gb = idx / HEAD_LANES;  // g * nb + ib
    const uint32_t ib = (uint32_t)(gb % nb);
    const uint32_t g = (uint32_t)(gb / nb);
    const uint32_t row = g * HEAD_LANES + lane;
    uint4 *dst = wq + gb * HEAD_CHUNKS * HEAD_LANES + lane;
    if (row >= rows) {
        for (int c = 0; c < HEAD_CHUNKS; ++c) dst[c * HEAD_LANES] = make_uint4(0, 0, 0, 0);
        wd[gb * HEAD_LANES + lane] = 0;
        return;
    }
    const uint8_t *b = src + ((uint64_t)row * nb + ib) * Q6K_BLOCK_BYTES;
    uint32_t words[48];
    for (int j = 0; j < 16; ++j) {
        uint32_t l0 = 0, l1 = 0, hw = 0;
        for (int e = 0; e < 4; ++e) {
            const uint32_t w0 = q6k_quant_at(b, 16 * j + e), w1 = q6k_quant_at(b, 16 * j + 4 + e);
            const uint32_t w2 = q6k_quant_at(b, 16 * j + 8 + e), w3 = q6k_quant_at(b, 16 * j + 12 + e);
            l0 |= ((w0 & 15) | ((w1 & 15) << 4)) << (8 * e);
            l1 |= ((w2 & 15) | ((w3 & 15) << 4)) << (8 * e);
            hw |= ((w0 >> 4) | ((w1 >> 4) << 2) | ((w2 >> 4) << 4) | ((w3 >> 4) << 6)) << (8 * e);
        }
        const int p = j >> 2, q = j & 3;
        // chunk 3p: {L0,L1} of sub-blocks 4p, 4p+1; chunk 3p+1: of 4p+2, 4p+3;
        // chunk 3p+2: H of 4p..4p+3.
        const int pair_word = 4 * (3 * p + (q >> 1)) + 2 * (q & 1);
        words[pair_word] = l0;
        words[pair_word + 1] = l1;
        words[4 * (3 * p + 2) + q] = hw;
    }
    for (int c = 0; c < 12; ++c)
        dst[c * HEAD_LANES] = make_uint4(words[4 * c], words[4 * c + 1], words[4 * c + 2], words[4 * c + 3]);
    uint32_t sc[4];
    for (int w = 0; w < 4; ++w)
        sc[w] = (uint32_t)b[192 + 4 * w] | ((uint32_t)b[193 + 4 * w] << 8) | ((uint32_t)b[194 + 4 * w] << 16) |
                ((uint32_t)b[195 + 4 * w] << 24);
    dst[12 * HEAD_LANES] = make_uint4(sc[0], sc[1], sc[2], sc[3]);
    wd[gb * HEAD_LANES + lane] = (uint16_t)(b[208] | (b[209] << 8));
}

// ------------------------------------------------------------ activations

// (v * id).round().clamp(-127, 127) as i8 (quant.rs:368-370): round half away
// from zero, NaN passes the clamp and converts to 0.
__device__ inline int quant_one(float v, float id) {
    const float r = roundf(v * id);
    float c = r < -127.0f ? -127.0f : r;
    c = c > 127.0f ? 127.0f : c;
    return c == c ? (int)c : 0;
}

// Activations::quantize_batch (quant.rs:337-375). One wave per (row, block);
// lane l holds values 4l..4l+3 of the block (zero past k, which the reference
// leaves out of the maximum and quantizes to 0). The maximum is order-free
// (f32::max ignores NaN; fmaxf does too), so a wave reduction gives the
// reference's amax. Writes the head's layout (`act`, may be null) and the
// reference's ActBlock fields (`out_d`, `out_qs`, `out_bsums`, each may be
// null).
__global__ __launch_bounds__(256) void k_quantize_rows(const float *__restrict__ x, uint32_t t, uint32_t k,
                                                       uint32_t nb, uint32_t *__restrict__ act,
                                                       float *__restrict__ out_d, int8_t *__restrict__ out_qs,
                                                       int16_t *__restrict__ out_bsums) {
    const uint32_t wave = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    const uint32_t lane = threadIdx.x & 63;
    if (wave >= t * nb) return;
    const uint32_t tt = wave / nb, ib = wave % nb;
    const float *src = x + (uint64_t)tt * k + (uint64_t)ib * QK;
    const uint32_t base = ib * QK + 4 * lane;
    float v[4];
    for (int e = 0; e < 4; ++e) v[e] = base + e < k ? src[4 * lane + e] : 0.0f;
    float amax = 0.0f;
    for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(v[e]));
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float d = amax / 127.0f;
    const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    int q[4];
    uint32_t packed = 0;
    for (int e = 0; e < 4; ++e) {
        q[e] = quant_one(v[e], id);
        packed |= ((uint32_t)q[e] & 0xFF) << (8 * e);
    }
    int bsum = q[0] + q[1] + q[2] + q[3];
    bsum += __shfl_xor(bsum, 1);
    bsum += __shfl_xor(bsum, 2);
    const uint64_t blk = (uint64_t)tt * nb + ib;
    if (act) {
        uint32_t *a = act + blk * ACT_WORDS;
        a[lane] = packed;
        if ((lane & 3) == 0) a[64 + lane / 4] = (uint32_t)(-32 * bsum);
        if (lane == 0) a[80] = __float_as_uint(d);
        if (lane >= 1 && lane <= 3) a[80 + lane] = 0;
    }
    if (out_qs) reinterpret_cast<uint32_t *>(out_qs + blk * QK)[lane] = packed;
    if (out_bsums && (lane & 3) == 0) out_bsums[blk * 16 + lane / 4] = (int16_t)bsum;
    if (out_d && lane == 0) out_d[blk] = d;
}

// ------------------------------------------------------------------- head

// The four activation-ordered weight dwords of a sub-block from its L0, L1, H.
__device__ inline void unpack_sub(uint32_t l0, uint32_t l1, uint32_t h, uint32_t &w0, uint32_t &w1, uint32_t &w2,
                                  uint32_t &w3) {
    w0 = (l0 & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
    w1 = ((l0 >> 4) & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
    w2 = (l1 & 0x0F0F0F0Fu) | (h & 0x30303030u);
    w3 = ((l1 >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
}

// Sign-extended low 24 bits: tells the compiler the operand fits v_mad_i32_i24.
// Every value passed here is within +/-2^17 (a sub-block dot).
__device__ inline int fits24(int v) { return (v << 8) >> 8; }

// One lane per vocabulary row, T activation rows per pass (t <= T active).
// The activation blocks of the pass sit in LDS; every lane reads the same
// words (broadcast). Per block: 13 coalesced 16-byte weight loads and the f16
// scale, the integer dots with v_dot4_i32_i8 (unsigned 6-bit weights < 128 are
// valid signed bytes; each sub-block's dot starts from -32 * bsum), then the
// reference's f32 line per token.
template <int T>
__global__ __launch_bounds__(HEAD_THREADS) void k_head_q6k(const uint4 *__restrict__ wq,
                                                            const uint16_t *__restrict__ wd,
                                                            const uint32_t *__restrict__ act, uint32_t t,
                                                            uint32_t nb, uint32_t rows, uint32_t groups,
                                                            float *__restrict__ out, uint64_t out_stride) {
    extern __shared__ uint4 sact4[];
    const uint32_t words = t * nb * ACT_WORDS;
    {
        const uint4 *src = reinterpret_cast<const uint4 *>(act);
        for (uint32_t i = threadIdx.x; i < words / 4; i += HEAD_THREADS) sact4[i] = src[i];
    }
    __syncthreads();
    const uint32_t *sact = reinterpret_cast<const uint32_t *>(sact4);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t g = blockIdx.x * HEAD_WAVES + threadIdx.x / 64;
    if (g >= groups) return;
    const uint4 *wp = wq + (uint64_t)g * nb * HEAD_CHUNKS * HEAD_LANES + lane;
    const uint16_t *dp = wd + (uint64_t)g * nb * HEAD_LANES + lane;

    float sum[T];
#pragma unroll
    for (int tt = 0; tt < T; ++tt) sum[tt] = 0.0f;

    for (uint32_t ib = 0; ib < nb; ++ib) {
        uint4 c[HEAD_CHUNKS];
#pragma unroll
        for (int i = 0; i < HEAD_CHUNKS; ++i) c[i] = wp[((uint64_t)ib * HEAD_CHUNKS + i) * HEAD_LANES];
        const float dw = __half2float(__ushort_as_half(dp[(uint64_t)ib * HEAD_LANES]));
        int isum[T];
#pragma unroll
        for (int tt = 0; tt < T; ++tt) isum[tt] = 0;
        const uint32_t scw[4] = {c[12].x, c[12].y, c[12].z, c[12].w};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint4 a = c[3 * p], b = c[3 * p + 1], hh = c[3 * p + 2];
            const uint32_t l0s[4] = {a.x, a.z, b.x, b.z};
            const uint32_t l1s[4] = {a.y, a.w, b.y, b.w};
            const uint32_t hs[4] = {hh.x, hh.y, hh.z, hh.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j = 4 * p + q;
                uint32_t w0, w1, w2, w3;
                unpack_sub(l0s[q], l1s[q], hs[q], w0, w1, w2, w3);
                const int sj = (int)(int8_t)(scw[p] >> (8 * q));
#pragma unroll
                for (int tt = 0; tt < T; ++tt) {
                    if (tt < (int)t) {
                        const uint32_t *ab = sact + ((uint64_t)tt * nb + ib) * ACT_WORDS;
                        const uint4 av = *reinterpret_cast<const uint4 *>(ab + 4 * j);
                        int dj = (int)ab[64 + j];
                        dj = __builtin_amdgcn_sdot4((int)w0, (int)av.x, dj, false);
                        dj = __builtin_amdgcn_sdot4((int)w1, (int)av.y, dj, false);
                        dj = __builtin_amdgcn_sdot4((int)w2, (int)av.z, dj, false);
                        dj = __builtin_amdgcn_sdot4((int)w3, (int)av.w, dj, false);
                        isum[tt] += sj * fits24(dj);
                    }
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            if (tt < (int)t) {
                const float ad = __uint_as_float(sact[((uint64_t)tt * nb + ib) * ACT_WORDS + 80]);
                const float scale = ad * dw;
                sum[tt] = sum[tt] + scale * (float)isum[tt];
            }
        }
    }
    const uint32_t row = g * HEAD_LANES + lane;
    if (row < rows) {
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
            if (tt < (int)t) out[(uint64_t)tt * out_stride + row] = sum[tt];
    }
}

}  // namespace rl
