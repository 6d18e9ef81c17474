// Trellis decode straight into v_mfma_f32_16x16x32_f16 B fragments.
//
// Fragment layout (checked on gfx950): B[k][n] of a 32 x 16 block, lane L holds n = L & 15 and
// k = 8 (L >> 4) + j for j = 0..7 as four packed fp16 pairs; A[m][k]: m = L & 15, same k; D[m][n]: n = L & 15,
// m = 4 (L >> 4) + i.
// One 32 x 16 B block = two vertically adjacent 16x16 tiles (tile-row 2s + (L >> 5)). Lane L needs column
// n of its tile and rows 8rh .. 8rh + 7 (rh = (L >> 4) & 1): chunk q = n & 7, positions u = o + u' with
// o = 2 rh + 4 (n >> 3) and u' in {0, 1, 8, 9, 16, 17, 24, 25}. The lane loads the few ring words covering those
// windows, funnel-shifts them by its (lane-dependent) bit offset so every window sits at a compile-time offset, and
// decodes its own 8 values: no value is decoded twice and no cross-lane exchange is needed.
#pragma once

#include "exl3_device.h"

namespace exl3 {

typedef float f4_t __attribute__((ext_vector_type(4)));

// Window of normalised position u' (bits [u'K, u'K + 16) of R), low 16 bits valid.
template <int K>
__device__ __forceinline__ uint32_t frag_window(const uint32_t* R, int up) {
    const int E = up * K + 16;
    const int IW = (E - 1) >> 5;
    const int SH = 32 * (IW + 1) - E;
    if (SH == 0) return R[IW];
    if (E - 16 >= 32 * IW) return R[IW] >> SH;
    return __builtin_amdgcn_alignbit(R[IW - 1], R[IW], SH);
}

// h values (1024 + bytesum, the codebook affine left out) of lane `lane`'s B fragment for the tile whose 8K ring
// words start at `tw`. Words are read with in-tile wrap-around, so every access stays inside the tile.
template <int K>
__device__ __forceinline__ h8_t frag_decode(const uint32_t* __restrict__ tw, int lane) {
    constexpr int W = 8 * K;
    constexpr int NW = (48 + 25 * K + 31) / 32;
    const int q = lane & 7, h = (lane >> 3) & 1, rh = (lane >> 4) & 1;
    const int start = (32 * q + 2 * rh + 4 * h + 1) * K - 16;   // first ring bit needed (-15 .. 256K)
    const int W0 = (start - 1) >> 5;                             // floor((start - 1) / 32), >= -1
    const uint32_t sh = (uint32_t)(32 - (start - 32 * W0));      // 0 .. 31
    uint32_t R[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        int w = W0 + i;
        w = w < 0 ? w + W : (w >= W ? w - W : w);
        R[i] = ldg_nt(tw + w);
    }
#pragma unroll
    for (int i = 0; i < NW - 1; ++i) R[i] = __builtin_amdgcn_alignbit(R[i], R[i + 1], sh);
    uint32_t p[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        p[c] = __builtin_bit_cast(uint32_t, mul1_pair_raw(frag_window<K>(R, 8 * c), frag_window<K>(R, 8 * c + 1)));
    typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
    u4_t v = {p[0], p[1], p[2], p[3]};
    return __builtin_bit_cast(h8_t, v);
}

// Split form of frag_decode for software pipelining: the ring-word indices a lane reads inside any tile do not
// depend on the tile, so they are computed once (frag_setup), words are loaded ahead (frag_load), and decoded later
// (frag_finish).
template <int K>
struct FragCfg {
    static constexpr int NW = (48 + 25 * K + 31) / 32;
    int widx[NW];
    uint32_t sh;
};

template <int K>
__device__ __forceinline__ void frag_setup(int lane, FragCfg<K>& c) {
    constexpr int W = 8 * K;
    const int q = lane & 7, h = (lane >> 3) & 1, rh = (lane >> 4) & 1;
    const int start = (32 * q + 2 * rh + 4 * h + 1) * K - 16;
    const int W0 = (start - 1) >> 5;
    c.sh = (uint32_t)(32 - (start - 32 * W0));
#pragma unroll
    for (int i = 0; i < FragCfg<K>::NW; ++i) {
        int w = W0 + i;
        c.widx[i] = w < 0 ? w + W : (w >= W ? w - W : w);
    }
}

template <int K>
__device__ __forceinline__ void frag_load(const uint32_t* __restrict__ tw, const FragCfg<K>& c,
                                          uint32_t (&R)[FragCfg<K>::NW]) {
#pragma unroll
    for (int i = 0; i < FragCfg<K>::NW; ++i) R[i] = ldg_nt(tw + c.widx[i]);
}

// First ring word (-1 .. 8K - 1) and funnel shift of lane `lane`'s fragment windows (see frag_decode).
template <int K>
__device__ __forceinline__ void frag_origin(int lane, int& w0, uint32_t& sh) {
    const int q = lane & 7, h = (lane >> 3) & 1, rh = (lane >> 4) & 1;
    const int start = (32 * q + 2 * rh + 4 * h + 1) * K - 16;
    w0 = (start - 1) >> 5;
    sh = (uint32_t)(32 - (start - 32 * w0));
}

template <int K>
__device__ __forceinline__ h8_t frag_finish(uint32_t (&R)[FragCfg<K>::NW], uint32_t sh) {
    constexpr int NW = FragCfg<K>::NW;
    uint32_t N[NW];
#pragma unroll
    for (int i = 0; i < NW - 1; ++i) N[i] = __builtin_amdgcn_alignbit(R[i], R[i + 1], sh);
    N[NW - 1] = R[NW - 1];
    uint32_t p[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        p[c] = __builtin_bit_cast(uint32_t, mul1_pair_raw(frag_window<K>(N, 8 * c), frag_window<K>(N, 8 * c + 1)));
    typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
    u4_t v = {p[0], p[1], p[2], p[3]};
    return __builtin_bit_cast(h8_t, v);
}

// k-permuted B fragments (K <= 5). Lane L = (n = L & 15, kg = L >> 4) takes tile-row kg >> 1 of the block and
// decodes two runs of four consecutive positions of its tile, t0 + {0..3} and t0 + 8 + {0..3} with
// t0 = 32 (n & 7) + 4 (n >> 3) + 16 (kg & 1): rows 4 (kg & 1) + {0, 1, 8, 9} and 4 (kg & 1) + {2, 3, 10, 11} of
// column n. Packed as rows 4 (kg & 1) + {0..3}, then 4 (kg & 1) + 8 + {0..3}, the lane's eight k are the 4-k units
// u = 4 (kg >> 1) + (kg & 1) and u + 2 of the 32-k block, so A must be staged with those two units side by side.
// A run's bits [(t + 1) K - 16, (t + 4) K) fit one funnel-shifted word (window i at bit 16 - i K), read from a staged
// slot laid out as [w(8K - 1), w(0) .. w(8K - 1), w(0), w(1), w(2)]: the funnel whose first bit is ring bit `a`
// (>= -15) takes slot words (a + 31) >> 5 and the next one, shifted by 31 - ((a + 31) & 31).
template <int K>
__device__ __forceinline__ void fragp_origin(int lane, int (&off)[2], uint32_t (&sh)[2]) {
    static_assert(K >= 1 && K <= 5, "k-permuted fragments need four windows in one funnel");
    const int n = lane & 15, kg = lane >> 4;
    const int t0 = 32 * (n & 7) + 4 * (n >> 3) + 16 * (kg & 1);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const int b = (t0 + 8 * g + 1) * K + 15;            // first bit + 31
        off[g] = b >> 5;
        sh[g] = (uint32_t)(~b & 31);
    }
}

// w[2g], w[2g + 1]: run g's two slot words
template <int K>
__device__ __forceinline__ h8_t fragp_finish(const uint32_t (&w)[4], const uint32_t (&sh)[2]) {
    uint32_t p[4];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const uint32_t F = __builtin_amdgcn_alignbit(w[2 * g], w[2 * g + 1], sh[g]);
        p[g] = __builtin_bit_cast(uint32_t, mul1_pair_raw(F >> 16, __builtin_amdgcn_ubfe(F, 16 - K, 16)));
        p[2 + g] = __builtin_bit_cast(
            uint32_t, mul1_pair_raw(__builtin_amdgcn_ubfe(F, 16 - 2 * K, 16), __builtin_amdgcn_ubfe(F, 16 - 3 * K, 16)));
    }
    typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
    u4_t v = {p[0], p[1], p[2], p[3]};
    return __builtin_bit_cast(h8_t, v);
}

// Per-tile K: dispatch on the tile's bitrate (all lanes of one tile take the same branch).
__device__ __forceinline__ h8_t frag_decode_k(const uint32_t* __restrict__ tw, int Kt, int lane) {
    switch (Kt) {
        case 1: return frag_decode<1>(tw, lane);
        case 2: return frag_decode<2>(tw, lane);
        case 3: return frag_decode<3>(tw, lane);
        case 4: return frag_decode<4>(tw, lane);
        case 5: return frag_decode<5>(tw, lane);
        case 6: return frag_decode<6>(tw, lane);
        case 7: return frag_decode<7>(tw, lane);
        case 8: return frag_decode<8>(tw, lane);
        default: {
            h8_t z = {};
            return z;
        }
    }
}

}  // namespace exl3
