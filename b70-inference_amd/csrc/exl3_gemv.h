// Decode-in-GEMV core shared by the dense linear and the grouped MoE kernels.
//
// A workgroup of 4 waves works on one 128-column strip of one projection over a k range made of whole Hadamard
// blocks (128 k = 8 tile-rows). The transformed activations of that range sit in LDS; each wave streams every 4th
// tile-row of the strip, decodes its 32 positions per lane in registers and accumulates sum_k a_k * h_k on the matrix
// cores (4x4x4 MFMA blocks; h = 1024 + bytesum, the codebook affine is applied once per output: c1 * acc +
// c2 * sum_k a_k).
#pragma once

#include "exl3_device.h"

namespace exl3 {

constexpr int kGemvKBMax = 8;        // Hadamard blocks (128 k) per workgroup split
constexpr int kGemvTargetWG = 1024;  // workgroups a GEMV launch aims for (256 CUs x 4); EXL3MI_TARGET_WG overrides
constexpr int kGemvMaxSplits = 8;    // k-splits of a launch with up to 2 rows, at most (twice that for more rows)
constexpr int kGemvMaxRows = 8;      // rows per GEMV pass
#ifndef EXL3_LINEAR_RING
#define EXL3_LINEAR_RING 3
#endif
constexpr int kLinearRing = EXL3_LINEAR_RING;   // register ring depth of the dense GEMV

// acc[m][h] += sum over tile-rows lt = lt0, lt0 + step, ... < nt of sum_r xs[m * xs_ld + 16 lt + r] * h(16 lt + r, col)
// where `sp` points at tile-row 0 of the strip, tile-rows are `rs` words apart, and lane l owns columns
// 16(l >> 3) + (l & 7) + 8h. Three register buffers in a ring: loads run two tile-rows ahead of the decode and every
// buffer is consumed in place, so a decode only waits for its own load.
//
// The products run on the matrix cores (EXL3_GEMV_MFMA, the default): v_mfma_f32_4x4x4_16b_f16 is 16 independent
// 4x4x4 products, block b = lanes 4b .. 4b + 3, D[lane 4b + j][i] = sum_k A[lane 4b + i][k] B[lane 4b + j][k]. A lane
// gives as A its own column's four decoded k of one row quad (two of its packed pairs: rows r, r + 1 and r + 2, r + 3
// of one column half, the same rows in every lane) and as B token (lane & 3)'s activations at those rows, so
// D[lane 4b + j][i] accumulates token j's product for lane 4b + i's column: eight 4x4x4 MFMAs per tile-row for up to
// four tokens (sixteen for up to eight) instead of 16 v_dot2 per token, and the VALU keeps only the decode. The
// accumulators are moved to the per-lane layout once, after the strip (quad broadcasts).
#ifndef EXL3_GEMV_MFMA
#define EXL3_GEMV_MFMA 1
#endif
#ifndef EXL3_GEMV_MFMA_MIN_ROWS
#define EXL3_GEMV_MFMA_MIN_ROWS 2
#endif
// one-row GEMVs keep v_dot2 (16 per tile-row): there the MFMA form is no clear win (4096 x 4096 linear -0.9 %, one-token
// 5376 x 21504 dense MLP -1.5 %, one-token top-10 decode layer of 512 experts +1.3 %); from two rows on it wins (two-row
// dense MLP -7 %, four-row -11 %)
template <int M>
constexpr bool gemv_mfma() { return EXL3_GEMV_MFMA && M >= EXL3_GEMV_MFMA_MIN_ROWS; }
typedef _Float16 gh4_t __attribute__((ext_vector_type(4)));
typedef float gf4_t __attribute__((ext_vector_type(4)));

template <int M>
struct GemvAcc {
    static constexpr int NG = (M + 3) / 4;                // token groups of 4
    gf4_t d[NG][2];                                       // [token group][column half]
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int g = 0; g < NG; ++g) d[g][0] = d[g][1] = gf4_t{0.f, 0.f, 0.f, 0.f};
    }
};

// decoded pairs of one tile-row: w[j] = rows (pos_row(2j), pos_row(2j) + 1) of column half pos_half(2j)
template <int K>
__device__ __forceinline__ void strip_tile_decode(const uint32_t (&D)[K], int lane, h2_t (&w)[16]) {
    uint32_t R[K + 1];
#pragma unroll
    for (int i = 0; i < K; ++i) R[1 + i] = D[i];
    chunk_prev<K>(lane, R);
    decode_chunk_raw<K>(R, w);
}

// Row quad q (rows 4q .. 4q + 3) of column half h is pairs (kQuadPair[q] + 2h, kQuadPair[q] + 2h + 4).
template <int M>
__device__ __forceinline__ void tile_row_mfma(const h2_t (&w)[16], int lane, const _Float16* xr, int xs_ld,
                                              GemvAcc<M>& acc) {
    constexpr int NG = GemvAcc<M>::NG;
    constexpr int kQuadPair[4] = {0, 8, 1, 9};
    gh4_t b[NG][4];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int tok = min(4 * g + (lane & 3), M - 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) b[g][q] = *reinterpret_cast<const gh4_t*>(xr + tok * xs_ld + 4 * q);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j1 = kQuadPair[q] + 2 * h, j2 = j1 + 4;
            const gh4_t a = {w[j1][0], w[j1][1], w[j2][0], w[j2][1]};
#pragma unroll
            for (int g = 0; g < NG; ++g) acc.d[g][h] = __builtin_amdgcn_mfma_f32_4x4x4f16(a, b[g][q], acc.d[g][h], 0, 0, 0);
        }
}

// value of lane (lane & ~3) + q (DPP quad_perm [q, q, q, q]; q a compile-time constant after unrolling)
__device__ __forceinline__ float quad_bcast(float v, int q) {
    const int u = __builtin_bit_cast(int, v);
    switch (q) {
        case 0: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, u, 0x00, 0xF, 0xF, false));
        case 1: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, u, 0x55, 0xF, 0xF, false));
        case 2: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, u, 0xAA, 0xF, 0xF, false));
        default: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, u, 0xFF, 0xF, 0xF, false));
    }
}

// out[m][h] += token m's sum for this lane's column: element (lane & 3) of lane (lane & ~3) + (m & 3) of d[m / 4][h]
template <int M>
__device__ __forceinline__ void gemv_acc_to_lanes(const GemvAcc<M>& acc, int lane, float (&out)[M][2]) {
    const int e = lane & 3;
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = quad_bcast(acc.d[m >> 2][h][i], m & 3);
            out[m][h] += e == 0 ? v[0] : e == 1 ? v[1] : e == 2 ? v[2] : v[3];
        }
}

template <int K, int M>
__device__ __forceinline__ void strip_tile_row(const uint32_t (&D)[K], int lane, const _Float16* xr, int xs_ld,
                                               float (&acc)[M][2]) {
    h2_t w[16];
    strip_tile_decode<K>(D, lane, w);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int r = pos_row(2 * j), h = pos_half(2 * j);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            h2_t xv = *reinterpret_cast<const h2_t*>(xr + m * xs_ld + r);
            acc[m][h] = __builtin_amdgcn_fdot2(w[j], xv, acc[m][h], false);
        }
    }
}

// Unconditional (the index is clamped to the last tile-row, nt > 0), so the waitcnt pass sees straight-line loads.
// Offsets are 32-bit word counts (a projection's trellis holds fewer than 2^32 words; the host checks).
// `base` is the lane's first chunk word in tile-row 0 (strip_lane_base); PL: PLANAR4 word order (WordOrder).
template <int K, bool PL = false>
__device__ __forceinline__ void strip_load(uint32_t (&D)[K], const uint32_t* __restrict__ base, uint32_t rs, int lt,
                                           int nt) {
    const uint32_t off = (uint32_t)(lt < nt ? lt : nt - 1) * rs;
#pragma unroll
    for (int i = 0; i < K; ++i) D[i] = ldg_nt(base + off + WordOrder<K, PL>::word_off(i));
    __builtin_amdgcn_sched_barrier(0);   // keep the prefetch where it is issued (the scheduler would sink it)
}

// The lane's first chunk word of a strip (8 consecutive tiles starting at a multiple of 4 tiles) at tile-row 0.
template <int K, bool PL = false>
__device__ __forceinline__ const uint32_t* strip_lane_base(const uint32_t* __restrict__ sp, int lane) {
    return sp + WordOrder<K, PL>::chunk_base(lane >> 3, lane & 7);
}

// Ring of R register buffers: buffer r holds tile-row i + r of the wave's rows lt0 + i * step; loads run R - 1 rows
// ahead of the decode. strip_prefetch issues the first R - 1 rows (so their latency overlaps whatever the caller
// does next); strip_gemv_run consumes them and streams the rest.
template <int K, int R>
struct StripRing {
    uint32_t D[R][K];
};

// With CHECK false the caller guarantees lt0 < nt: the loads are then issued without a branch, so the wait counts of
// loads issued before them stay exact (a branch around them makes the compiler drain every load at the join).
template <int K, int R, bool CHECK = true, bool PL = false>
__device__ __forceinline__ void strip_prefetch(const uint32_t* __restrict__ sp, size_t rs, int lt0, int nt, int step,
                                               int lane, StripRing<K, R>& ring) {
    if (CHECK && lt0 >= nt) return;
    const uint32_t* base = strip_lane_base<K, PL>(sp, lane) + (size_t)lt0 * rs;
    const int n = (nt - lt0 + step - 1) / step;
#pragma unroll
    for (int r = 0; r < R - 1; ++r) strip_load<K, PL>(ring.D[r], base, (uint32_t)(rs * step), r, n);
}

template <int K, int M, int R, bool PL = false>
__device__ __forceinline__ void strip_gemv_run(const uint32_t* __restrict__ sp, size_t rs, int lt0, int nt, int step,
                                               int lane, const _Float16* xs, int xs_ld, float (&acc)[M][2],
                                               StripRing<K, R>& ring) {
    if (lt0 >= nt) return;
    const int n = (nt - lt0 + step - 1) / step;          // tile-rows of this wave: lt0 + i * step, i < n
    const uint32_t* base = strip_lane_base<K, PL>(sp, lane) + (size_t)lt0 * rs;
    const uint32_t rstep = (uint32_t)(rs * step);
    GemvAcc<M> ma;
    if constexpr (gemv_mfma<M>()) ma.zero();
    auto tile_row = [&](int r, int i) {
        const _Float16* xr = xs + (lt0 + i * step) * 16;
        if constexpr (gemv_mfma<M>()) {
            h2_t w[16];
            strip_tile_decode<K>(ring.D[r], lane, w);
            tile_row_mfma<M>(w, lane, xr, xs_ld, ma);
        } else {
            strip_tile_row<K, M>(ring.D[r], lane, xr, xs_ld, acc);
        }
    };
    int i = 0;
    for (; i + R <= n; i += R) {                         // branch-free body: loads stay R - 1 tile-rows ahead
#pragma unroll
        for (int r = 0; r < R; ++r) {
            strip_load<K, PL>(ring.D[(r + R - 1) % R], base, rstep, i + r + R - 1, n);
            tile_row(r, i + r);
        }
    }
#pragma unroll
    for (int r = 0; r < R - 1; ++r)
        if (i + r < n) tile_row(r, i + r);
    if constexpr (gemv_mfma<M>()) gemv_acc_to_lanes<M>(ma, lane, acc);
}

template <int K, int M>
__device__ __forceinline__ void strip_gemv(const uint32_t* __restrict__ sp, size_t rs, int lt0, int nt, int step,
                                           int lane, const _Float16* xs, int xs_ld, float (&acc)[M][2]) {
    StripRing<K, 3> ring;
    strip_prefetch<K, 3>(sp, rs, lt0, nt, step, lane, ring);
    strip_gemv_run<K, M, 3>(sp, rs, lt0, nt, step, lane, xs, xs_ld, acc, ring);
}

// Per-tile K (mixed bitrate): tile i of the projection (row-major over [k/16, n/16]) holds 8 * kmap[i] words at
// words + woff[i]. A wave still covers 8 consecutive tiles of a tile-row; lanes branch on their tile's K (all lanes
// of one tile take the same branch, so the cross-lane `prev` permute stays inside the branch).
template <int K, int M>
__device__ __forceinline__ void mixed_tile_row(const uint32_t* __restrict__ tw, int lane, const _Float16* xr,
                                               int xs_ld, float (&acc)[M][2]) {
    uint32_t D[K];
    const uint32_t* q = tw + (lane & 7) * K;
#pragma unroll
    for (int i = 0; i < K; ++i) D[i] = ldg_nt(q + i);
    strip_tile_row<K, M>(D, lane, xr, xs_ld, acc);
}

template <int K>
__device__ __forceinline__ void mixed_tile_decode(const uint32_t* __restrict__ tw, int lane, h2_t (&w)[16]) {
    uint32_t D[K];
    const uint32_t* q = tw + (lane & 7) * K;
#pragma unroll
    for (int i = 0; i < K; ++i) D[i] = ldg_nt(q + i);
    strip_tile_decode<K>(D, lane, w);
}

template <int M>
__device__ __forceinline__ void strip_gemv_mixed(const uint32_t* __restrict__ words, const uint8_t* __restrict__ kmap,
                                                 const int32_t* __restrict__ woff, int tn, int tile_n0, int tr0,
                                                 int lt0, int nt, int step, int lane, const _Float16* xs, int xs_ld,
                                                 float (&acc)[M][2]) {
    GemvAcc<M> ma;
    if constexpr (gemv_mfma<M>()) ma.zero();
    for (int lt = lt0; lt < nt; lt += step) {
        const int tile = (tr0 + lt) * tn + tile_n0 + (lane >> 3);
        const int Kt = ldg(kmap + tile);
        const uint32_t* tw = words + ldg(woff + tile);
        const _Float16* xr = xs + lt * 16;
        if constexpr (gemv_mfma<M>()) {
            h2_t w[16];                                  // decoded per lane (the 8 lanes of a tile share a case);
            switch (Kt) {                                // the MFMAs run after the lanes reconverge
                case 1: mixed_tile_decode<1>(tw, lane, w); break;
                case 2: mixed_tile_decode<2>(tw, lane, w); break;
                case 3: mixed_tile_decode<3>(tw, lane, w); break;
                case 4: mixed_tile_decode<4>(tw, lane, w); break;
                case 5: mixed_tile_decode<5>(tw, lane, w); break;
                case 6: mixed_tile_decode<6>(tw, lane, w); break;
                case 7: mixed_tile_decode<7>(tw, lane, w); break;
                default: mixed_tile_decode<8>(tw, lane, w); break;
            }
            tile_row_mfma<M>(w, lane, xr, xs_ld, ma);
        } else {
            switch (Kt) {
                case 1: mixed_tile_row<1, M>(tw, lane, xr, xs_ld, acc); break;
                case 2: mixed_tile_row<2, M>(tw, lane, xr, xs_ld, acc); break;
                case 3: mixed_tile_row<3, M>(tw, lane, xr, xs_ld, acc); break;
                case 4: mixed_tile_row<4, M>(tw, lane, xr, xs_ld, acc); break;
                case 5: mixed_tile_row<5, M>(tw, lane, xr, xs_ld, acc); break;
                case 6: mixed_tile_row<6, M>(tw, lane, xr, xs_ld, acc); break;
                case 7: mixed_tile_row<7, M>(tw, lane, xr, xs_ld, acc); break;
                case 8: mixed_tile_row<8, M>(tw, lane, xr, xs_ld, acc); break;
                default: break;
            }
        }
    }
    if constexpr (gemv_mfma<M>()) gemv_acc_to_lanes<M>(ma, lane, acc);
}

// ------------------------------------------------------------------------------------------------ split-K handoff
// Workgroups of one output strip publish fp32 partials; the last to arrive (per-strip counter) reduces them.
// Partials are written with agent-scope relaxed atomic stores (write-through past the XCD-local L2) and read with
// agent-scope atomic loads, and every wave drains its stores (s_waitcnt) before the arrival atomic. This avoids the
// device-scope fence, which on gfx950 writes back the whole L2 of the XCD once per workgroup.
#ifndef EXL3_SPLITK_FENCE
#define EXL3_SPLITK_FENCE 0
#endif

__device__ __forceinline__ void splitk_store(float* p, float v) {
#if EXL3_SPLITK_FENCE
    *p = v;
#else
    __hip_atomic_store((__attribute__((address_space(1))) float*)p, v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
#endif
}

__device__ __forceinline__ float splitk_load(const float* p) {
    return __hip_atomic_load((const __attribute__((address_space(1))) float*)p, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Returns true in every thread of the last-arriving workgroup (of `nparts`); that workgroup resets the counter
// when it is done (splitk_reset), so counters are zero between launches.
__device__ __forceinline__ bool splitk_arrive(int* cnt, int nparts, int* s_flag) {
#if EXL3_SPLITK_FENCE
    __threadfence();
#else
    __builtin_amdgcn_s_waitcnt(0);     // this wave's partial stores have completed
#endif
    __syncthreads();
    if (threadIdx.x == 0) {
        int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = (old == nparts - 1);
    }
    __syncthreads();
    bool last = *s_flag;
#if EXL3_SPLITK_FENCE
    if (last) __threadfence();
#endif
    return last;
}

// Input transform of one 128-block for one row by one wave, in two parts so that a caller can issue the loads early:
// had_in_load loads the block's x and sign elements lane and lane + 64 (unconditional loads: x must point at readable
// memory); had_in_finish writes fp16(H128(fp16(x * suh)) / sqrt(128)) at elements lane and lane + 64 to dst[lane],
// dst[lane + 64], with x taken as zeros unless `valid`, and returns the block's element sum (every lane gets it).
struct HadIn {
    uint16_t xa, xb, sa, sb;
};
__device__ __forceinline__ HadIn had_in_load(const uint16_t* __restrict__ x, const uint16_t* __restrict__ suh, int lane) {
    return HadIn{ldg(x + lane), ldg(x + lane + 64), ldg(suh + lane), ldg(suh + lane + 64)};
}
__device__ __forceinline__ float had_in_finish(const HadIn& v, bool valid, _Float16* dst, int lane) {
    float va = (float)(_Float16)(h2f(v.xa) * h2f(v.sa));
    float vb = (float)(_Float16)(h2f(v.xb) * h2f(v.sb));
    va = valid ? va : 0.f;
    vb = valid ? vb : 0.f;
    fwht128_wave(va, vb, lane);
    _Float16 ha = (_Float16)(va * kRsqrt128), hb = (_Float16)(vb * kRsqrt128);
    dst[lane] = ha;
    dst[lane + 64] = hb;
    return wave_sum_f32((float)ha + (float)hb);
}

}  // namespace exl3
