// Device-side building blocks of the EXL3 trellis kernels for gfx950 (CDNA4, wave64).
//
// Tile format (ext-op-inventory.md:717-733; glm/xpu/csrc/exl3_esimd.h:4-14): a 16x16 tile of K-bit codes is 8K
// little-endian uint32 words = one MSB-first ring of 256K bits. Position t (0..255) decodes the 16-bit window of ring
// bits [(t+1)K - 16, (t+1)K) (circular) and lands at row 8((t>>1)&1) + 2((t>>3)&3) + (t&1) (input / k index),
// column (t>>5) + 8((t>>2)&1) (output / n index).
//
// Lane chunking used by every kernel here: a wave covers a strip of 8 consecutive tiles of one tile-row (128 output
// columns). Lane l owns chunk q = l & 7 of tile l >> 3: the K words [Kq, Kq + K) of that tile, i.e. exactly the 32
// positions t = 32q .. 32q + 31, which are columns q and q + 8 over all 16 rows. The strip is 64K contiguous words,
// lane l reading words [Kl, Kl + K): one fully coalesced K-dword load per lane per tile-row, for every K. The only
// other bits a lane needs are the up-to-15 bits before its chunk: the last word of lane l - 1, or (q == 0) of
// lane l + 7 (the ring wraps inside the tile), fetched with one cross-lane permute.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exl3 {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kMul1 = 0x83DCD12Du;
constexpr float kRsqrt128 = 0.08838834764831845f;

// Loads through explicit global (address space 1) pointers. Pointers that reach a kernel through tables or
// descriptors are generic to the compiler, which would emit flat loads; flat loads also count against the LDS
// counter, so every wait on them becomes a full drain and software prefetching stops working.
template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));

template <typename T>
__device__ __forceinline__ T ldg_nt(const T* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) T*)p);
}

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// ------------------------------------------------------------------------------------------------ windows

// State (in the low 16 bits; upper bits are garbage) of position u (0..31) of the lane's chunk.
// R[0] is the word before the chunk, R[1..K] the chunk's words. In R's bit string the chunk starts at bit 32, so
// position u's window is bits [16 + (u+1)K, 32 + (u+1)K). All offsets are compile-time after unrolling.
template <int K>
__device__ __forceinline__ uint32_t window_raw(const uint32_t* R, int u) {
    const int E = 32 + (u + 1) * K;        // exclusive end bit
    const int IW = (E - 1) >> 5;           // word holding the last bit
    const int SH = 32 * (IW + 1) - E;      // right shift that aligns the window end with bit 0
    if (SH == 0) return R[IW];
    if (E - 16 >= 32 * IW) return R[IW] >> SH;
    return __builtin_amdgcn_alignbit(R[IW - 1], R[IW], SH);
}

// mul1 codebook for two states (low 16 bits used), packed fp16 pair (lo = s0, hi = s1).
// x = s * 0x83DCD12D mod 2^32; 0x6400 + bytesum(x) is the fp16 bit pattern of 1024 + bytesum(x) (sad_u8 adds the
// four unsigned bytes, sad_hi_u8 adds them into the high half); w = fma(h, 0x1EEE, 0xC931) in fp16, one rounding:
// bit-exact with the reference decode (glm/xpu/csrc/exl3_esimd.h:46-68).
__device__ __forceinline__ h2_t mul1_pair(uint32_t s0, uint32_t s1) {
    uint32_t x0 = (s0 & 0xFFFFu) * kMul1;
    uint32_t x1 = (s1 & 0xFFFFu) * kMul1;
    uint32_t h = __builtin_amdgcn_sad_hi_u8(x1, 0u, __builtin_amdgcn_sad_u8(x0, 0u, 0x64006400u));
    const h2_t c1 = {(_Float16)0.00676727294921875f, (_Float16)0.00676727294921875f};
    const h2_t c2 = {(_Float16)-10.3828125f, (_Float16)-10.3828125f};
    return __builtin_elementwise_fma(__builtin_bit_cast(h2_t, h), c1, c2);
}

// The same without the affine: packed fp16 pair of h = 1024 + bytesum(x) (exact integers). A dot product over
// decoded weights is then sum_k a_k w_k = c1 * sum_k a_k h_k + c2 * sum_k a_k (the reference's fold,
// glm/xpu/csrc/exl3_esimd.h:82-91); kernels apply c1 and c2 once per output instead of once per weight.
constexpr float kMul1C1 = 0.00676727294921875f, kMul1C2 = -10.3828125f;
__device__ __forceinline__ h2_t mul1_pair_raw(uint32_t s0, uint32_t s1) {
    uint32_t x0 = (s0 & 0xFFFFu) * kMul1;
    uint32_t x1 = (s1 & 0xFFFFu) * kMul1;
    return __builtin_bit_cast(h2_t, __builtin_amdgcn_sad_hi_u8(x1, 0u, __builtin_amdgcn_sad_u8(x0, 0u, 0x64006400u)));
}

// row (k index inside the tile) and column half (0: column q, 1: column q + 8) of chunk position u
__host__ __device__ constexpr int pos_row(int u) { return 8 * ((u >> 1) & 1) + 2 * ((u >> 3) & 3) + (u & 1); }
__host__ __device__ constexpr int pos_half(int u) { return (u >> 2) & 1; }

// Word order of a tile-row. Tile order (PL false): tile t's 8K words at 8K t. PLANAR4 (PL true; the reference's
// expert blobs, glm/xpu/exl3xpu/moe_offload.py:68-78, glm/xpu/pack_store.py:35-54): a tile's words are G periods of
// D = K / gcd(K, 32) words, and within every group of 4 consecutive tiles word (tile t, period g, plane i) sits at
// 4G i + G t + g (G = 8K / D); D = 1 (K = 1, 2, 4, 8) is tile order. Word j of a lane's chunk q (tile word Kq + j) is
// period q gcd + j / D, plane j % D. So both orders read a lane's K chunk words at
//   group base + tile-in-group * G + q * gcd + word_off(j)
// with G = 8K, gcd = K, word_off(j) = j in tile order: one K-dword load there, K dword loads at fixed offsets in
// PLANAR4 (coalesced across the lanes of a plane).
template <int K, bool PL>
struct WordOrder {
    static constexpr int GC = PL ? (K & -K) : K;         // gcd(K, 32) for K <= 8
    static constexpr int D = K / GC;
    static constexpr int G = 8 * K / D;
    static_assert(K >= 1 && K <= 8, "K in 1..8");
    __host__ __device__ static constexpr int word_off(int j) { return (j % D) * 4 * G + j / D; }
    // first word of chunk q of tile `tile` of a tile-row (tile counted from the row's first tile)
    __host__ __device__ static constexpr int chunk_base(int tile, int q) {
        return (tile & ~3) * 8 * K + (tile & 3) * G + q * GC;
    }
};

// Load the lane's K chunk words of one tile-row strip and the word before the chunk. `p` points at the strip's
// first word; returns R[0..K].
template <int K, bool PL = false>
__device__ __forceinline__ void load_chunk(const uint32_t* __restrict__ p, int lane, uint32_t* R) {
    typedef WordOrder<K, PL> O;
    const uint32_t* q = p + O::chunk_base(lane >> 3, lane & 7);
#pragma unroll
    for (int i = 0; i < K; ++i) R[1 + i] = ldg_nt(q + O::word_off(i));
}

// R[0] = last word of the previous chunk of the lane's tile: lane l - 1, or l + 7 for chunk 0 (the ring wraps inside
// the 8 lanes of a tile; both stay inside the lane's 16-lane row, so two DPP row shifts do it).
template <int K>
__device__ __forceinline__ void chunk_prev(int lane, uint32_t* R) {
    const int v = (int)R[K];
    const int dn = __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1 (lane - 1)
    const int up = __builtin_amdgcn_update_dpp(0, v, 0x107, 0xF, 0xF, false);   // row_shl:7 (lane + 7)
    R[0] = (uint32_t)((lane & 7) ? dn : up);
}

// Decode the lane's 32 positions into 16 packed fp16 pairs: pair j holds positions (2j, 2j+1), i.e. rows
// (pos_row(2j), pos_row(2j)+1) of column half pos_half(2j).
// Window of position u (low 16 bits valid) given the funnel-shifted words N[j] = bits [32 j + 16, 32 j + 48) of R's
// bit string: a window inside one word of R is a shift of it; one that crosses the boundary at bit 32 IW lies inside
// N[IW - 1]. Either way one shift-and-mask (v_bfe_u32), the funnel shift being shared by every window crossing that
// boundary (about 16 / K of them) instead of one v_alignbit plus a mask per window.
// At K = 8 every window is byte-aligned and a crossing one is a single v_perm_b32 already: window_raw is kept there.
template <int K>
__device__ __forceinline__ uint32_t window_norm(const uint32_t* R, const uint32_t* N, int u) {
    if constexpr (K == 8) return window_raw<K>(R, u);
    const int E = 32 + (u + 1) * K;        // exclusive end bit
    const int IW = (E - 1) >> 5;           // word holding the last bit
    const int SH = 32 * (IW + 1) - E;
    if (E - 16 >= 32 * IW) return SH == 0 ? R[IW] : R[IW] >> SH;
    return N[IW - 1] >> (32 * IW + 16 - E);
}

template <int K>
__device__ __forceinline__ void funnel_words(const uint32_t* R, uint32_t* N) {
#pragma unroll
    for (int j = 0; j < K; ++j) N[j] = __builtin_amdgcn_alignbit(R[j], R[j + 1], 16);
}

template <int K>
__device__ __forceinline__ void decode_chunk(const uint32_t* R, h2_t* w) {
    uint32_t N[K];
    funnel_words<K>(R, N);
#pragma unroll
    for (int j = 0; j < 16; ++j) w[j] = mul1_pair(window_norm<K>(R, N, 2 * j), window_norm<K>(R, N, 2 * j + 1));
}

// Same positions, codebook affine left out (h = 1024 + bytesum).
template <int K>
__device__ __forceinline__ void decode_chunk_raw(const uint32_t* R, h2_t* w) {
    uint32_t N[K];
    funnel_words<K>(R, N);
#pragma unroll
    for (int j = 0; j < 16; ++j)
        w[j] = mul1_pair_raw(window_norm<K>(R, N, 2 * j), window_norm<K>(R, N, 2 * j + 1));
}

// ------------------------------------------------------------------------------------------------ Hadamard

// Value of lane (lane ^ M) (gfx950): DPP quad permutes for 1 and 2, row shifts for 4 (left or right by 4 inside the
// 16-lane row, by bit 2), a row rotate by 8 for 8, and v_permlane16/32_swap for 16 and 32 (swapping a register with
// itself: element [0] holds the lower partner row / half in the upper one, [1] the upper partner in the lower one).
template <int M>
__device__ __forceinline__ float lane_xor(float v, int lane) {
    const int u = __builtin_bit_cast(int, v);
    if constexpr (M == 1) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, u, 0xB1, 0xF, 0xF, false));
    if constexpr (M == 2) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, u, 0x4E, 0xF, 0xF, false));
    if constexpr (M == 4) {
        const int l = __builtin_amdgcn_update_dpp(0, u, 0x104, 0xF, 0xF, false);   // row_shl:4 (lane + 4)
        const int r = __builtin_amdgcn_update_dpp(0, u, 0x114, 0xF, 0xF, false);   // row_shr:4 (lane - 4)
        return __builtin_bit_cast(float, (lane & 4) ? r : l);
    }
    if constexpr (M == 8) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, u, 0x128, 0xF, 0xF, false));
    if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)u, (unsigned)u, false, false);
        return __builtin_bit_cast(float, (lane & 16) ? r[0] : r[1]);
    }
    if constexpr (M == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)u, (unsigned)u, false, false);
        return __builtin_bit_cast(float, (lane & 32) ? r[0] : r[1]);
    }
    return v;
}

template <int M>
__device__ __forceinline__ void fwht_stage(float& a, float& b, int lane) {
    const float pa = lane_xor<M>(a, lane), pb = lane_xor<M>(b, lane);
    const bool hi = lane & M;
    a = hi ? pa - a : a + pa;
    b = hi ? pb - b : b + pb;
}

// Unnormalised natural-order Sylvester FWHT-128 across a wave: lane l holds elements l (a) and l + 64 (b).
__device__ __forceinline__ void fwht128_wave(float& a, float& b, int lane) {
    const float s = a + b, d = a - b;
    a = s;
    b = d;
    fwht_stage<1>(a, b, lane);
    fwht_stage<2>(a, b, lane);
    fwht_stage<4>(a, b, lane);
    fwht_stage<8>(a, b, lane);
    fwht_stage<16>(a, b, lane);
    fwht_stage<32>(a, b, lane);
}

// ------------------------------------------------------------------------------------------------ wave reductions
// DPP reductions over the 64 lanes of a wave (gfx9 row_bcast form): xor 1 and xor 2 inside quads, mirrors inside
// half-rows and rows, then row_bcast15 / row_bcast31 across rows; lane 63 ends with the result, read back uniformly.
#define EXL3_DPP(v, ctrl, rmask) \
    (uint32_t) __builtin_amdgcn_update_dpp((int)ident, (int)(v), ctrl, rmask, 0xF, false)

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    const uint32_t ident = 0u;
    v = max(v, EXL3_DPP(v, 0xB1, 0xF));    // quad_perm [1,0,3,2]
    v = max(v, EXL3_DPP(v, 0x4E, 0xF));    // quad_perm [2,3,0,1]
    v = max(v, EXL3_DPP(v, 0x141, 0xF));   // row_half_mirror
    v = max(v, EXL3_DPP(v, 0x140, 0xF));   // row_mirror
    v = max(v, EXL3_DPP(v, 0x142, 0xA));   // row_bcast:15 into rows 1, 3
    v = max(v, EXL3_DPP(v, 0x143, 0xC));   // row_bcast:31 into rows 2, 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    const uint32_t ident = 0xFFFFFFFFu;
    v = min(v, EXL3_DPP(v, 0xB1, 0xF));
    v = min(v, EXL3_DPP(v, 0x4E, 0xF));
    v = min(v, EXL3_DPP(v, 0x141, 0xF));
    v = min(v, EXL3_DPP(v, 0x140, 0xF));
    v = min(v, EXL3_DPP(v, 0x142, 0xA));
    v = min(v, EXL3_DPP(v, 0x143, 0xC));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ float wave_sum_f32(float f) {
    const uint32_t ident = 0u;   // +0.0f
    uint32_t v = __builtin_bit_cast(uint32_t, f);
#define EXL3_ADD(ctrl, rmask) \
    v = __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, v) + __builtin_bit_cast(float, EXL3_DPP(v, ctrl, rmask)))
    EXL3_ADD(0xB1, 0xF);
    EXL3_ADD(0x4E, 0xF);
    EXL3_ADD(0x141, 0xF);
    EXL3_ADD(0x140, 0xF);
    EXL3_ADD(0x142, 0xA);
    EXL3_ADD(0x143, 0xC);
#undef EXL3_ADD
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane((int)v, 63));
}
#undef EXL3_DPP

// Order-preserving map of a float to uint32 (larger float -> larger key; NaN payloads sort above +inf).
__device__ __forceinline__ uint32_t float_key(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inverse of float_key.
__device__ __forceinline__ float key_float(uint32_t k) {
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ float h2f(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }
__device__ __forceinline__ uint16_t f2h(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }

}  // namespace exl3
