// The output head on gfx950: logits = token_embd (Q6_K, [k, rows]) times the
// normed hidden rows, bit-identical to rust-llm's CPU head
// (crates/rust-llm/src/forward.rs:932-937 → forward.rs:1157-1180 →
// crates/rust-llm/src/pool.rs:468-506 → crates/llm-core/src/kernels/mod.rs:273-300).
//
// What the bits depend on. The reference quantizes each activation row in
// blocks of 256 to int8 with one f32 scale per block (quant.rs:337-375), then
// per (token, vocabulary row) sums, block by block from 0.0 in f32,
//     (act.d * w.d) * (float)isum,   isum = sum_i s_{i/16} * (q_i - 32) * a_i,
// where isum is an exact i32. Any way of forming isum exactly gives the same
// bits; the f32 line is kept as it is, in block order.
//
// How isum is formed here: on the matrix cores, in f16 with f32 accumulation,
// exactly. Each sub-block scale s (an i8) is split as s = 16 * s_hi + s_lo with
// s_lo in [0, 15] and s_hi in [-8, 7]. Two products are accumulated over the
// block's 256 values with v_mfma_f32_16x16x32_f16:
//     D_lo = sum s_lo * (q - 32) * a,   D_hi = sum s_hi * (q - 32) * a.
// Every operand is an integer an f16 holds exactly (|s_lo (q-32)| <= 480,
// |s_hi (q-32)| <= 256, |a| <= 127), every product is exact in f32, and every
// partial sum is an integer below 2^24 (at most 256 * 480 * 127 < 15.7e6), so
// the accumulation is exact in any order. Then (float)isum = fl(16 * D_hi +
// D_lo), one fused multiply-add of the two exact integers.
//
// Layouts in HBM (built once by k_q6k_repack from the GGUF bytes), for a
// vocabulary of `groups` groups of 64 rows, each group four tiles of 16 rows:
//   Lane l = 16 h + m of a tile holds row m and the quarter h of each block:
//   values k = 64 h + 8 s + e (step s = 0..7, e = 0..7). The same k order is
//   used for the activations, so the matrix-core sum runs over the block.
//   wq  uint4 [nb][groups][4][3][64]: the lane's 64 unsigned 6-bit quants
//       (ggml's value before the -32), 48 bytes in the packing below.
//   ws  u32   [nb][groups][4][64]: the lane's four sub-block scales (i8),
//       sub-blocks 4h .. 4h+3; step s uses byte s / 2.
//   wd  u16   [nb][groups][4][16]: the f16 block scale of each row.
//   Total bytes equal the GGUF tensor's: 210 per row and block.
//   Packing of steps 2p and 2p+1 (values v0..v7 and v8..v15) in words
//   P0, P1, P2 = words 3p .. 3p+2, as 16-bit halves (low, high):
//     P0 = {v0 | v2 << 6 | (v12 & 15) << 12,  v1 | v3 << 6 | (v13 & 15) << 12}
//     P1 = {v4 | v6 << 6 | (v14 & 15) << 12,  v5 | v7 << 6 | (v15 & 15) << 12}
//     P2 = {v8 | v10 << 6 | (v12 >> 4) << 12 | (v14 >> 4) << 14,
//           v9 | v11 << 6 | (v13 >> 4) << 12 | (v15 >> 4) << 14}
//   so each f16 pair (v_2i, v_2i+1) comes out with a mask and an OR of the
//   f16 exponent bits (0x6400 | q is the f16 1024 + q).
//   Activations: int8 quants [Tcap][nb][256] and f32 scales [Tcap][nb], the
//   reference's ActBlock fields.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_device.h"

namespace rl {

constexpr int QK = 256;              // values per quantization block (quant.rs:12)
constexpr int Q6K_BLOCK_BYTES = 210; // ql 128, qh 64, scales 16, d f16 (quant.rs:19)
constexpr int HEAD_TILE = 16;        // vocabulary rows per matrix-core tile
constexpr int HEAD_TILES = 4;        // tiles per wave
constexpr int HEAD_GROUP = HEAD_TILE * HEAD_TILES;  // rows per wave
constexpr int HEAD_QCH = 3;          // 16-byte quant chunks per lane, tile and block
constexpr int HEAD_WAVES = 4;        // waves per workgroup
constexpr int HEAD_THREADS = HEAD_WAVES * 64;
constexpr int HEAD_NTILE = 16;       // activation rows per matrix-core column tile
constexpr int HEAD_MAX_NT = 2;       // column tiles one pass takes (32 rows)

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

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

// One thread per (block, group, tile, lane); lanes are innermost so the stores
// of a wave are contiguous. Rows at or past `rows` are zero.
__global__ void k_q6k_repack(const uint8_t *__restrict__ src, uint32_t rows, uint32_t nb, uint32_t groups,
                             uint4 *__restrict__ wq, uint32_t *__restrict__ ws, uint16_t *__restrict__ wd) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t total = (uint64_t)nb * groups * HEAD_TILES * 64;
    if (idx >= total) return;
    const uint32_t lane = (uint32_t)(idx & 63);
    const uint64_t bgt = idx >> 6;  // (ib * groups + g) * 4 + tw
    const uint32_t tw = (uint32_t)(bgt % HEAD_TILES);
    const uint64_t bg = bgt / HEAD_TILES;
    const uint32_t g = (uint32_t)(bg % groups);
    const uint32_t ib = (uint32_t)(bg / groups);
    const uint32_t m = lane & 15, h = lane >> 4;
    const uint32_t row = g * HEAD_GROUP + tw * HEAD_TILE + m;
    uint4 *dq = wq + bgt * HEAD_QCH * 64 + lane;
    if (row >= rows) {
        for (int c = 0; c < HEAD_QCH; ++c) dq[c * 64] = make_uint4(0, 0, 0, 0);
        ws[bgt * 64 + lane] = 0;
        if (h == 0) wd[bgt * HEAD_TILE + m] = 0;
        return;
    }
    const uint8_t *b = src + ((uint64_t)row * nb + ib) * Q6K_BLOCK_BYTES;
    uint32_t words[12];
    for (int p = 0; p < 4; ++p) {
        uint32_t v[16];
        for (int i = 0; i < 16; ++i) v[i] = q6k_quant_at(b, 64 * h + 16 * p + i);
        const uint32_t lo0 = v[0] | v[2] << 6 | (v[12] & 15) << 12, hi0 = v[1] | v[3] << 6 | (v[13] & 15) << 12;
        const uint32_t lo1 = v[4] | v[6] << 6 | (v[14] & 15) << 12, hi1 = v[5] | v[7] << 6 | (v[15] & 15) << 12;
        const uint32_t lo2 = v[8] | v[10] << 6 | (v[12] >> 4) << 12 | (v[14] >> 4) << 14;
        const uint32_t hi2 = v[9] | v[11] << 6 | (v[13] >> 4) << 12 | (v[15] >> 4) << 14;
        words[3 * p] = lo0 | hi0 << 16;
        words[3 * p + 1] = lo1 | hi1 << 16;
        words[3 * p + 2] = lo2 | hi2 << 16;
    }
    for (int c = 0; c < HEAD_QCH; ++c)
        dq[c * 64] = make_uint4(words[4 * c], words[4 * c + 1], words[4 * c + 2], words[4 * c + 3]);
    const uint8_t *sc = b + 192 + 4 * h;
    ws[bgt * 64 + lane] = (uint32_t)sc[0] | (uint32_t)sc[1] << 8 | (uint32_t)sc[2] << 16 | (uint32_t)sc[3] << 24;
    if (h == 0) wd[bgt * HEAD_TILE + m] = (uint16_t)(b[208] | (b[209] << 8));
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

// One activation block quantized by one wave (quant.rs:360-374): lane l holds
// values 4l..4l+3 (zero past `valid`, which the reference leaves out of the
// maximum and quantizes to 0). The maximum is order-free (f32::max ignores
// NaN; fmaxf does too), so a wave reduction gives the reference's amax.
// Returns the block scale, the lane's four quants packed little-endian, and
// the sum of the 16 quants of the lane's sub-block (in every lane of it).
__device__ inline float quantize_block_wave(const float *__restrict__ src, uint32_t valid, uint32_t lane,
                                            uint32_t &packed, int &bsum) {
    float v[4];
    for (int e = 0; e < 4; ++e) v[e] = 4 * lane + e < valid ? src[4 * lane + e] : 0.0f;
    float amax = 0.0f;
    for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(v[e]));
    amax = wave_maxnum_f32(amax);
    const float d = amax / 127.0f;
    const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    int q[4];
    packed = 0;
    for (int e = 0; e < 4; ++e) {
        q[e] = quant_one(v[e], id);
        packed |= ((uint32_t)q[e] & 0xFF) << (8 * e);
    }
    bsum = q[0] + q[1] + q[2] + q[3];
    bsum += (int)lane_xor<1>((uint32_t)bsum);
    bsum += (int)lane_xor<2>((uint32_t)bsum);
    return d;
}

// The dot path's byte order: bytes 1 and 2 of every word swapped, the order
// the unpacked weights come out in.
__device__ inline uint32_t dot_order(uint32_t packed) { return __builtin_amdgcn_perm(packed, packed, 0x03010200u); }

__device__ inline h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }

// Four signed int8 activations as two f16 pairs: bytes + 128 under the f16
// exponent of 1024, minus 1152, exact.
__device__ inline void act_pairs(uint32_t w, uint32_t &lo, uint32_t &hi) {
    const uint32_t u = w ^ 0x80808080u;
    const h2_t bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    lo = __builtin_bit_cast(uint32_t, as_h2(a) + bias);
    hi = __builtin_bit_cast(uint32_t, as_h2(b) + bias);
}

// The activation fragments of each 16-row tile and block, the matrix core's B
// operand in f16 (exact: the quants are integers in [-127, 127]): entry
// ((tile * nb + ib) * 8 + s) * 64 + 16 h + m holds activation row 16 tile + m,
// values 64 h + 8 s .. + 7 of block ib, in order.
constexpr int HEAD_FRAG_UINT4 = 8 * 64;  // uint4 per (tile, block)

// Activations::quantize_batch (quant.rs:337-375). One wave per (row, block).
// Writes the reference's ActBlock fields and the block's f16 fragments; each
// output may be null.
__global__ __launch_bounds__(256) void k_quantize_rows(const float *__restrict__ x, uint32_t t, uint32_t k,
                                                       uint32_t nb, float *__restrict__ out_d,
                                                       int8_t *__restrict__ out_qs,
                                                       int16_t *__restrict__ out_bsums,
                                                       uint4 *__restrict__ out_frag) {
    const uint32_t wave = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    const uint32_t lane = threadIdx.x & 63;
    if (wave >= t * nb) return;
    const uint32_t tt = wave / nb, ib = wave % nb;
    const uint32_t valid = k - ib * QK < QK ? k - ib * QK : QK;
    uint32_t packed;
    int bsum;
    const float d = quantize_block_wave(x + (uint64_t)tt * k + (uint64_t)ib * QK, valid, lane, packed, bsum);
    const uint64_t blk = (uint64_t)tt * nb + ib;
    if (out_qs) reinterpret_cast<uint32_t *>(out_qs + blk * QK)[lane] = packed;
    if (out_bsums && (lane & 3) == 0) out_bsums[blk * 16 + lane / 4] = (int16_t)bsum;
    if (out_d && lane == 0) out_d[blk] = d;
    if (out_frag) {
        // Values 64 h + 8 s .. + 7 are lanes 16 h + 2 s and the next one's.
        const uint32_t next = lane_xor<1>(packed);
        if ((lane & 1) == 0) {
            uint32_t p0, p1, p2, p3;
            act_pairs(packed, p0, p1);
            act_pairs(next, p2, p3);
            const uint32_t h = lane >> 4, s = (lane & 15) >> 1;
            out_frag[((uint64_t)(tt >> 4) * nb + ib) * HEAD_FRAG_UINT4 + s * 64 + 16 * h + (tt & 15)] =
                make_uint4(p0, p1, p2, p3);
        }
    }
}

// ------------------------------------------------------------------- head

// Sign-extended low 24 bits: tells the compiler the operand fits v_mad_i32_i24.
// Every value passed here is within +/-2^17 (a sub-block dot).
__device__ inline int fits24(int v) { return (v << 8) >> 8; }



// The masks of the unpacking, held in registers: gfx9 VOP3 takes no literal,
// so with the constants in registers each field is one v_and_or_b32.
struct UnpackConsts {
    uint32_t m6, m4, m2, mag;
};

__device__ inline UnpackConsts unpack_consts() {
    UnpackConsts c;
    asm volatile("v_mov_b32 %0, 0x003F003F" : "=v"(c.m6));
    asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(c.m4));
    asm volatile("v_mov_b32 %0, 0x00300030" : "=v"(c.m2));
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(c.mag));
    return c;
}

// The eight f16 pairs (1024 + q) of steps 2p and 2p+1 from P0, P1, P2.
__device__ inline void unpack_steps(uint32_t p0, uint32_t p1, uint32_t p2, uint32_t x[8], const UnpackConsts &k) {
    x[0] = (p0 & k.m6) | k.mag;
    x[1] = ((p0 >> 6) & k.m6) | k.mag;
    x[2] = (p1 & k.m6) | k.mag;
    x[3] = ((p1 >> 6) & k.m6) | k.mag;
    x[4] = (p2 & k.m6) | k.mag;
    x[5] = ((p2 >> 6) & k.m6) | k.mag;
    x[6] = ((p0 >> 12) & k.m4) | (((p2 >> 8) & k.m2) | k.mag);
    x[7] = ((p1 >> 12) & k.m4) | (((p2 >> 10) & k.m2) | k.mag);
}


// One tile's weights for one block: the lane's quant words, scale bytes and the
// f16 scales of rows 4h .. 4h+3.
struct HeadTile {
    uint4 q[HEAD_QCH];
    uint32_t sc;
    uint2 dd;
};

__device__ inline HeadTile load_tile(const uint4 *__restrict__ wq, const uint32_t *__restrict__ ws,
                                     const uint16_t *__restrict__ wd, uint64_t bgt, uint32_t lane, uint32_t h) {
    HeadTile r;
#pragma unroll
    for (int c = 0; c < HEAD_QCH; ++c) r.q[c] = wq[(bgt * HEAD_QCH + c) * 64 + lane];
    r.sc = ws[bgt * 64 + lane];
    r.dd = reinterpret_cast<const uint2 *>(wd + bgt * HEAD_TILE)[h];
    return r;
}

// Copies one block's activation fragments (HEAD_FRAG_UINT4 per column tile,
// written by k_quantize_rows) into LDS, cooperatively, with the block scale
// of each activation row.
template <int NT>
__device__ inline void fill_act(uint4 *__restrict__ frag, float *__restrict__ fd, const uint4 *__restrict__ af,
                                const float *__restrict__ ad, uint32_t nb, uint32_t ib) {
    for (uint32_t e = threadIdx.x; e < NT * HEAD_FRAG_UINT4; e += HEAD_THREADS) {
        const uint32_t nt = e / HEAD_FRAG_UINT4;
        frag[e] = af[((uint64_t)nt * nb + ib) * HEAD_FRAG_UINT4 + e % HEAD_FRAG_UINT4];
    }
    if (threadIdx.x < NT * HEAD_NTILE) fd[threadIdx.x] = ad[(uint64_t)threadIdx.x * nb + ib];
}

// One wave per group of 64 vocabulary rows (four 16-row tiles); NT column
// tiles of 16 activation rows. The workgroup walks the blocks in step (one
// barrier per block): the activation fragments of block ib + 1 are built in
// LDS while block ib is computed. Each tile takes 16 matrix-core products per
// column tile (8 steps, s_lo and s_hi) and then the reference's f32 line; the
// next tile's weights are in flight meanwhile. Four waves per SIMD: the
// fragments are read from LDS step by step, and a scheduling barrier per step
// pair keeps the compiler from hoisting every step's reads (which costs the
// registers of a fourth wave). `stab` is the per-scale-byte table {s_lo,
// -1056 s_lo, s_hi, -1056 s_hi} as f16 pairs, so (1024 + q) * s + c =
// (q - 32) * s exactly in one packed FMA.
template <int NT>
__global__ __launch_bounds__(HEAD_THREADS) __attribute__((amdgpu_waves_per_eu(4)))
void k_head_mfma_lds(const uint4 *__restrict__ wq, const uint32_t *__restrict__ ws, const uint16_t *__restrict__ wd,
                const uint4 *__restrict__ af, const float *__restrict__ ad, uint32_t t, uint32_t nb,
                uint32_t rows, uint32_t groups, float *__restrict__ out, uint64_t out_stride) {
    __shared__ uint4 stab[256];
    __shared__ uint4 frag[2][NT * 8 * 64];
    __shared__ float fd[2][NT * HEAD_NTILE];
    {
        const int s = (int)(int8_t)threadIdx.x;  // HEAD_THREADS == 256 entries
        const int slo = s & 15, shi = s >> 4;
        const h2_t lo = {(_Float16)(float)slo, (_Float16)(float)slo};
        const h2_t clo = {(_Float16)(float)(-1056 * slo), (_Float16)(float)(-1056 * slo)};
        const h2_t hi = {(_Float16)(float)shi, (_Float16)(float)shi};
        const h2_t chi = {(_Float16)(float)(-1056 * shi), (_Float16)(float)(-1056 * shi)};
        stab[threadIdx.x & 255] = make_uint4(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, clo),
                                             __builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, chi));
    }
    fill_act<NT>(frag[0], fd[0], af, ad, nb, 0);
    const uint32_t lane = threadIdx.x & 63;
    // Wave-uniform, so weight addresses are a scalar base plus the lane offset.
    const uint32_t g = __builtin_amdgcn_readfirstlane(blockIdx.x * HEAD_WAVES + threadIdx.x / 64);
    // A wave past the vocabulary still takes part in the barriers.
    const bool active = g < groups;
    const uint32_t gg = active ? g : groups - 1;
    const uint32_t m = lane & 15, h = lane >> 4;
    const UnpackConsts uk = unpack_consts();

    f4_t sum[NT][HEAD_TILES];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int tw = 0; tw < HEAD_TILES; ++tw) sum[nt][tw] = f4_t{0.f, 0.f, 0.f, 0.f};

    HeadTile cur = load_tile(wq, ws, wd, (uint64_t)gg * HEAD_TILES, lane, h);
    for (uint32_t ib = 0; ib < nb; ++ib) {
        __syncthreads();  // block ib's fragments are built; block ib - 1's buffer is free
        if (ib + 1 < nb) fill_act<NT>(frag[(ib + 1) & 1], fd[(ib + 1) & 1], af, ad, nb, ib + 1);
        const uint4 *bfr = frag[ib & 1];
        float adn[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) adn[nt] = fd[ib & 1][nt * HEAD_NTILE + m];
        const uint32_t nxt_ib = ib + 1 < nb ? ib + 1 : ib;  // past the end: re-read (a cache hit)
#pragma unroll
        for (int tw = 0; tw < HEAD_TILES; ++tw) {
            // The next tile: tile tw + 1 of this block, or the first of the next.
            const uint64_t nbgt = tw + 1 < HEAD_TILES ? ((uint64_t)ib * groups + gg) * HEAD_TILES + tw + 1
                                                      : ((uint64_t)nxt_ib * groups + gg) * HEAD_TILES;
            const HeadTile nxt = load_tile(wq, ws, wd, nbgt, lane, h);
            const uint32_t w12[12] = {cur.q[0].x, cur.q[0].y, cur.q[0].z, cur.q[0].w, cur.q[1].x, cur.q[1].y,
                                      cur.q[1].z, cur.q[1].w, cur.q[2].x, cur.q[2].y, cur.q[2].z, cur.q[2].w};
            f4_t acc_lo[NT], acc_hi[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                acc_lo[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
                acc_hi[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                __builtin_amdgcn_sched_barrier(0);
                uint32_t x[8];
                unpack_steps(w12[3 * p], w12[3 * p + 1], w12[3 * p + 2], x, uk);
                const uint4 st = stab[(cur.sc >> (8 * p)) & 255];
                const h2_t slo = as_h2(st.x), clo = as_h2(st.y), shi = as_h2(st.z), chi = as_h2(st.w);
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    h2_t lo[4], hi[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        lo[e] = __builtin_elementwise_fma(as_h2(x[4 * u + e]), slo, clo);
                        hi[e] = __builtin_elementwise_fma(as_h2(x[4 * u + e]), shi, chi);
                    }
                    const h8_t alo = {lo[0][0], lo[0][1], lo[1][0], lo[1][1], lo[2][0], lo[2][1], lo[3][0], lo[3][1]};
                    const h8_t ahi = {hi[0][0], hi[0][1], hi[1][0], hi[1][1], hi[2][0], hi[2][1], hi[3][0], hi[3][1]};
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const h8_t b = __builtin_bit_cast(h8_t, bfr[(nt * 8 + 2 * p + u) * 64 + lane]);
                        acc_lo[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b, acc_lo[nt], 0, 0, 0);
                        acc_hi[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b, acc_hi[nt], 0, 0, 0);
                    }
                }
            }
            // Rows 4h + i of the tile, activation row nt*16 + m.
            const uint32_t dw2[2] = {cur.dd.x, cur.dd.y};
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // (float)isum: 16 D_hi + D_lo is formed exactly (both are
                    // integers below 2^24) and rounded once.
                    const float fisum = __builtin_fmaf(acc_hi[nt][i], 16.0f, acc_lo[nt][i]);
                    const float dw = __half2float(__ushort_as_half((uint16_t)(dw2[i >> 1] >> (16 * (i & 1)))));
                    const float scale = adn[nt] * dw;
                    sum[nt][tw][i] = sum[nt][tw][i] + scale * fisum;
                }
            }
            cur = nxt;
        }
    }
    if (!active) return;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t n = nt * HEAD_NTILE + m;
        if (n >= t) continue;
#pragma unroll
        for (int tw = 0; tw < HEAD_TILES; ++tw)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t row = g * HEAD_GROUP + tw * HEAD_TILE + 4 * h + i;
                if (row < rows) out[(uint64_t)n * out_stride + row] = sum[nt][tw][i];
            }
    }
}

// One wave per group of 64 vocabulary rows (four 16-row tiles); NT column
// tiles of 16 activation rows. Per block: the activation fragments are
// converted once and reused by the four tiles; per tile, 16 matrix-core
// products (8 steps, s_lo and s_hi) and the reference's f32 line. The next
// tile's weights (and, at the last tile, the next block's) are in flight while
// a tile is computed. `stab` is the per-scale-byte table {s_lo, -1056 s_lo,
// s_hi, -1056 s_hi} as f16 pairs, so (1024 + q) * s + c = (q - 32) * s exactly
// in one packed FMA.
template <int NT>
__global__ __launch_bounds__(HEAD_THREADS) __attribute__((amdgpu_waves_per_eu(NT == 1 ? 4 : 2)))
void k_head_mfma_regs(const uint4 *__restrict__ wq,
                                                               const uint32_t *__restrict__ ws,
                                                               const uint16_t *__restrict__ wd,
                                                               const uint4 *__restrict__ af,
                                                               const float *__restrict__ ad, uint32_t t,
                                                               uint32_t nb, uint32_t rows, uint32_t groups,
                                                               float *__restrict__ out, uint64_t out_stride) {
    __shared__ uint4 stab[256];
    {
        const int s = (int)(int8_t)threadIdx.x;  // HEAD_THREADS == 256 entries
        const int slo = s & 15, shi = s >> 4;
        const h2_t lo = {(_Float16)(float)slo, (_Float16)(float)slo};
        const h2_t clo = {(_Float16)(float)(-1056 * slo), (_Float16)(float)(-1056 * slo)};
        const h2_t hi = {(_Float16)(float)shi, (_Float16)(float)shi};
        const h2_t chi = {(_Float16)(float)(-1056 * shi), (_Float16)(float)(-1056 * shi)};
        stab[threadIdx.x & 255] = make_uint4(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, clo),
                                             __builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, chi));
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t g = __builtin_amdgcn_readfirstlane(blockIdx.x * HEAD_WAVES + threadIdx.x / 64);
    if (g >= groups) return;
    const uint32_t m = lane & 15, h = lane >> 4;
    const UnpackConsts uk = unpack_consts();

    f4_t sum[NT][HEAD_TILES];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int tw = 0; tw < HEAD_TILES; ++tw) sum[nt][tw] = f4_t{0.f, 0.f, 0.f, 0.f};

    HeadTile cur = load_tile(wq, ws, wd, (uint64_t)g * HEAD_TILES, lane, h);
    for (uint32_t ib = 0; ib < nb; ++ib) {
        const uint32_t nxt_ib = ib + 1 < nb ? ib + 1 : ib;  // the last block re-reads itself (a cache hit)
        // The block's activation fragments, as k_quantize_rows wrote them.
        h8_t bf[NT][8];
        float adn[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            adn[nt] = ad[(uint64_t)(nt * HEAD_NTILE + m) * nb + ib];
            const uint4 *fp = af + ((uint64_t)nt * nb + ib) * HEAD_FRAG_UINT4 + lane;
#pragma unroll
            for (int st = 0; st < 8; ++st) bf[nt][st] = __builtin_bit_cast(h8_t, fp[st * 64]);
        }
#pragma unroll
        for (int tw = 0; tw < HEAD_TILES; ++tw) {
            const uint64_t nbgt = tw + 1 < HEAD_TILES ? ((uint64_t)ib * groups + g) * HEAD_TILES + tw + 1
                                                      : ((uint64_t)nxt_ib * groups + g) * HEAD_TILES;
            const HeadTile nxt = load_tile(wq, ws, wd, nbgt, lane, h);
            const uint32_t w12[12] = {cur.q[0].x, cur.q[0].y, cur.q[0].z, cur.q[0].w, cur.q[1].x, cur.q[1].y,
                                      cur.q[1].z, cur.q[1].w, cur.q[2].x, cur.q[2].y, cur.q[2].z, cur.q[2].w};
            f4_t acc_lo[NT], acc_hi[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                acc_lo[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
                acc_hi[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                uint32_t x[8];
                unpack_steps(w12[3 * p], w12[3 * p + 1], w12[3 * p + 2], x, uk);
                const uint4 st = stab[(cur.sc >> (8 * p)) & 255];
                const h2_t slo = as_h2(st.x), clo = as_h2(st.y), shi = as_h2(st.z), chi = as_h2(st.w);
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    h2_t lo[4], hi[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        lo[e] = __builtin_elementwise_fma(as_h2(x[4 * u + e]), slo, clo);
                        hi[e] = __builtin_elementwise_fma(as_h2(x[4 * u + e]), shi, chi);
                    }
                    const h8_t alo = {lo[0][0], lo[0][1], lo[1][0], lo[1][1], lo[2][0], lo[2][1], lo[3][0], lo[3][1]};
                    const h8_t ahi = {hi[0][0], hi[0][1], hi[1][0], hi[1][1], hi[2][0], hi[2][1], hi[3][0], hi[3][1]};
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        acc_lo[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bf[nt][2 * p + u], acc_lo[nt], 0, 0, 0);
                        acc_hi[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bf[nt][2 * p + u], acc_hi[nt], 0, 0, 0);
                    }
                }
            }
            // Rows 4h + i of the tile, activation row nt*16 + m.
            const uint32_t dw2[2] = {cur.dd.x, cur.dd.y};
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // (float)isum: 16 D_hi + D_lo is formed exactly (both are
                    // integers below 2^24) and rounded once.
                    const float fisum = __builtin_fmaf(acc_hi[nt][i], 16.0f, acc_lo[nt][i]);
                    const float dw = __half2float(__ushort_as_half((uint16_t)(dw2[i >> 1] >> (16 * (i & 1)))));
                    const float scale = adn[nt] * dw;
                    sum[nt][tw][i] = sum[nt][tw][i] + scale * fisum;
                }
            }
            cur = nxt;
        }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t n = nt * HEAD_NTILE + m;
        if (n >= t) continue;
#pragma unroll
        for (int tw = 0; tw < HEAD_TILES; ++tw)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t row = g * HEAD_GROUP + tw * HEAD_TILE + 4 * h + i;
                if (row < rows) out[(uint64_t)n * out_stride + row] = sum[nt][tw][i];
            }
    }
}

// The dot path, for one or two activation rows: v_dot4_i32_i8 on the same
// layout, with the activation rows quantized by the workgroup itself into LDS
// (the same arithmetic as k_quantize_rows). Lane (m, h) unpacks its
// quarter-block to bytes (unsigned 6-bit weights, which are valid signed
// bytes) in the order [v0 v2 v1 v3] per word, dots them with the activation
// words in that order starting from -32 * bsum of the sub-block, scales by the
// sub-block scale, and the four lanes of a row add their exact partial sums
// with two lane shuffles. Then the reference's f32 line; lane (m, h) stores
// activation row h. LDS per activation block: 64 words of quants, 16 words of
// -32 * bsum, the f32 scale, 3 words of padding.
constexpr int DOT_ACT_WORDS = 84;

template <int T>
__global__ __launch_bounds__(HEAD_THREADS) __attribute__((amdgpu_waves_per_eu(4)))
void k_head_dot(const uint4 *__restrict__ wq, const uint32_t *__restrict__ ws, const uint16_t *__restrict__ wd,
                const float *__restrict__ x, uint32_t k, uint32_t nb, uint32_t rows, uint32_t groups,
                float *__restrict__ out, uint64_t out_stride) {
    extern __shared__ uint4 sact4[];
    uint32_t *sact = reinterpret_cast<uint32_t *>(sact4);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x / 64;
    const uint32_t g = __builtin_amdgcn_readfirstlane(blockIdx.x * HEAD_WAVES + wave);
    const uint32_t gg = g < groups ? g : groups - 1;
    const uint32_t m = lane & 15, h = lane >> 4;
    const uint32_t M6 = 0x003F003Fu, M6S = 0x3F003F00u, M4 = 0x000F000Fu, M2 = 0x00300030u, M4S = 0x0F000F00u,
                   M2S = 0x30003000u;

    // The first tile's weights are in flight while the activations are quantized.
    const uint64_t tile0 = (uint64_t)gg * HEAD_TILES;
    HeadTile cur = load_tile(wq, ws, wd, tile0, lane, h);
    uint16_t curd = wd[tile0 * HEAD_TILE + m];
    for (uint32_t w = wave; w < T * nb; w += HEAD_WAVES) {
        const uint32_t tt = w / nb, ib = w % nb;
        const uint32_t valid = k - ib * QK < QK ? k - ib * QK : QK;
        uint32_t packed;
        int bsum;
        const float d = quantize_block_wave(x + (uint64_t)tt * k + (uint64_t)ib * QK, valid, lane, packed, bsum);
        uint32_t *a = sact + (uint64_t)w * DOT_ACT_WORDS;
        a[lane] = dot_order(packed);
        if ((lane & 3) == 0) a[64 + lane / 4] = (uint32_t)(-32 * bsum);
        if (lane == 0) a[80] = __float_as_uint(d);
    }
    __syncthreads();
    if (g >= groups) return;

    float sum[HEAD_TILES][T];
#pragma unroll
    for (int tw = 0; tw < HEAD_TILES; ++tw)
#pragma unroll
        for (int tt = 0; tt < T; ++tt) sum[tw][tt] = 0.0f;

    for (uint32_t ib = 0; ib < nb; ++ib) {
        const uint32_t nxt_ib = ib + 1 < nb ? ib + 1 : ib;  // past the end: re-read (a cache hit)
        uint4 a[T][4];
        uint4 cv[T];
        float adv[T];
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            const uint32_t *ab = sact + ((uint64_t)tt * nb + ib) * DOT_ACT_WORDS;
#pragma unroll
            for (int c = 0; c < 4; ++c) a[tt][c] = reinterpret_cast<const uint4 *>(ab + 16 * h)[c];
            cv[tt] = reinterpret_cast<const uint4 *>(ab + 64)[h];
            adv[tt] = __uint_as_float(ab[80]);
        }
#pragma unroll
        for (int tw = 0; tw < HEAD_TILES; ++tw) {
            const uint64_t nbgt = tw + 1 < HEAD_TILES ? ((uint64_t)ib * groups + g) * HEAD_TILES + tw + 1
                                                      : ((uint64_t)nxt_ib * groups + g) * HEAD_TILES;
            const HeadTile nxt = load_tile(wq, ws, wd, nbgt, lane, h);
            const uint16_t nxtd = wd[nbgt * HEAD_TILE + m];
            const uint32_t w12[12] = {cur.q[0].x, cur.q[0].y, cur.q[0].z, cur.q[0].w, cur.q[1].x, cur.q[1].y,
                                      cur.q[1].z, cur.q[1].w, cur.q[2].x, cur.q[2].y, cur.q[2].z, cur.q[2].w};
            int isum[T];
#pragma unroll
            for (int tt = 0; tt < T; ++tt) isum[tt] = 0;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t p0 = w12[3 * p], p1 = w12[3 * p + 1], p2 = w12[3 * p + 2];
                const uint32_t b0 = (p0 & M6) | ((p0 << 2) & M6S);
                const uint32_t b1 = (p1 & M6) | ((p1 << 2) & M6S);
                const uint32_t b2 = (p2 & M6) | ((p2 << 2) & M6S);
                const uint32_t b3 = ((p0 >> 12) & M4) | ((p2 >> 8) & M2) | ((p1 >> 4) & M4S) | ((p2 >> 2) & M2S);
                const int sj = (int)(int8_t)(cur.sc >> (8 * p));
#pragma unroll
                for (int tt = 0; tt < T; ++tt) {
                    const uint32_t av[4] = {a[tt][p].x, a[tt][p].y, a[tt][p].z, a[tt][p].w};
                    const uint32_t cw[4] = {cv[tt].x, cv[tt].y, cv[tt].z, cv[tt].w};
                    int dsum = (int)cw[p];
                    dsum = __builtin_amdgcn_sdot4((int)b0, (int)av[0], dsum, false);
                    dsum = __builtin_amdgcn_sdot4((int)b1, (int)av[1], dsum, false);
                    dsum = __builtin_amdgcn_sdot4((int)b2, (int)av[2], dsum, false);
                    dsum = __builtin_amdgcn_sdot4((int)b3, (int)av[3], dsum, false);
                    isum[tt] += sj * fits24(dsum);
                }
            }
            const float dw = __half2float(__ushort_as_half(curd));
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
                int v = isum[tt];
                v += (int)lane_xor<16>((uint32_t)v);
                v += (int)lane_xor<32>((uint32_t)v);
                const float scale = adv[tt] * dw;
                sum[tw][tt] = sum[tw][tt] + scale * (float)v;
            }
            cur = nxt;
            curd = nxtd;
        }
    }
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
        if (h != (uint32_t)tt) continue;
#pragma unroll
        for (int tw = 0; tw < HEAD_TILES; ++tw) {
            const uint32_t row = g * HEAD_GROUP + tw * HEAD_TILE + m;
            if (row < rows) out[(uint64_t)tt * out_stride + row] = sum[tw][tt];
        }
    }
}

// ------------------------------------------------------------ embedding lookup

// The reference's embedding lookup (forward.rs:1127-1138), dequantize_row's
// Q6_K arm (quant.rs:177-203), from the repacked tensor: value i of a row is
// d * (float)(s * (q - 32)), the integer product exact and one f32 multiply,
// as the reference forms it. One thread per (token, block, quarter h, step
// pair p): the row's 16 values 64 h + 16 p .. + 15 of the block, all of
// sub-block 4 h + p, from words 3p .. 3p+2 of lane 16 h + m's quant chunks (the
// packing above). A token at or past `rows` gives a row of NaN: the reference
// asserts (forward.rs:1130-1134), which a kernel cannot.
constexpr int EMBED_THREADS = 256;

__global__ __launch_bounds__(EMBED_THREADS) void k_embed_rows(const uint4 *__restrict__ wq,
                                                              const uint32_t *__restrict__ ws,
                                                              const uint16_t *__restrict__ wd,
                                                              const uint32_t *__restrict__ tokens, uint32_t t,
                                                              uint32_t k, uint32_t nb, uint32_t rows, uint32_t groups,
                                                              float *__restrict__ out, uint64_t out_stride) {
    const uint64_t idx = (uint64_t)blockIdx.x * EMBED_THREADS + threadIdx.x;
    if (idx >= (uint64_t)t * nb * 16) return;
    const uint32_t p = (uint32_t)(idx & 3), h = (uint32_t)((idx >> 2) & 3);
    const uint64_t tb = idx >> 4;
    const uint32_t ib = (uint32_t)(tb % nb), ti = (uint32_t)(tb / nb);
    const uint32_t k0 = ib * QK + 64 * h + 16 * p;
    if (k0 >= k) return;
    const uint32_t n = k - k0 < 16 ? k - k0 : 16;
    float *o = out + (uint64_t)ti * out_stride + k0;
    const uint32_t tok = tokens[ti];
    float v[16];
    if (tok >= rows) {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = __builtin_nanf("");
    } else {
        const uint32_t g = tok / HEAD_GROUP, tw = (tok / HEAD_TILE) % HEAD_TILES, m = tok % HEAD_TILE;
        const uint64_t bgt = ((uint64_t)ib * groups + g) * HEAD_TILES + tw;
        const uint32_t lane = 16 * h + m;
        const uint32_t *q = reinterpret_cast<const uint32_t *>(wq + bgt * HEAD_QCH * 64 + lane);
        uint32_t pw[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const uint32_t wi = 3 * p + j;
            pw[j] = q[(wi / 4) * 64 * 4 + wi % 4];
        }
        const int s = (int)(int8_t)(ws[bgt * 64 + lane] >> (8 * p));
        const float d = __half2float(__ushort_as_half(wd[bgt * HEAD_TILE + m]));
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            const uint32_t a = pw[0] >> (16 * x), b = pw[1] >> (16 * x), c = pw[2] >> (16 * x);
            const uint32_t u[8] = {a & 63, (a >> 6) & 63, b & 63, (b >> 6) & 63,
                                   c & 63, (c >> 6) & 63, ((a >> 12) & 15) | ((c >> 12) & 3) << 4,
                                   ((b >> 12) & 15) | ((c >> 14) & 3) << 4};
            // u[j] is value 2 j + x of the sixteen.
#pragma unroll
            for (int j = 0; j < 8; ++j) v[2 * j + x] = d * (float)(s * ((int)u[j] - 32));
        }
    }
    if (n == 16 && (reinterpret_cast<uintptr_t>(o) & 15) == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            reinterpret_cast<float4 *>(o)[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if ((uint32_t)i < n) o[i] = v[i];
    }
}

}  // namespace rl
