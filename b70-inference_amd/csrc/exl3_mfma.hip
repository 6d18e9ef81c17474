// Expert-sorted ragged grouped GEMM on fp16 MFMA for prefill-sized calls.
//
// Rows (token, expert pairs) are grouped by expert and cut into blocks of up to kMfmaRows rows; in a prefill call
// every expert with rows gets blocks (no GEMV items). Per layer call:
//   pairs_had   transformed gate / up inputs of every block row, xh[pair][proj] = fp16(H128(fp16(x * suh)) / sqrt(128)),
//               and their 128-blocks' sums (the codebook affine term)
//   gateup      workgroup per (block, 128-column block of I), full H; each wave owns two gate and two up tile columns
//               and decodes them straight into MFMA B fragments once per 32-k step (B holds h = 1024 + bytesum; the
//               affine is applied as c1 * acc + c2 * rowsum(A) in the epilogue), then the fused activation / down-input
//               epilogue (Hadamard * svh, act, * suh_d, Hadamard) per 16-row group
//   down        workgroup per (block, 256-column block of H), full I, epilogue Hadamard * svh_d * w, then the combine
// The A rows of the active row groups are staged through a four-stage LDS ring (loaded into registers four steps
// ahead, stored two steps ahead), weight words three steps ahead; one barrier every second step. Workgroup ids are laid out so that the column blocks
// of one row block run on one XCD (shared L2 for its A rows).
// Semantics: the reference's GateUpDpasKernel / DownDpasKernel / moe_prefill (glm/xpu/csrc/exl3_moe.n128.sycl:
// 472-689, 868-916) and exllamav3's exl3_moe (ext-op-inventory.md:1060-1093).
#include "exl3_device.h"
#include "exl3_gemv.h"
#include "exl3_mfma.h"
#include "exl3_moe.h"
#include "exl3_moe_dev.h"
#include "exl3_runtime.h"

namespace exl3 {

// ------------------------------------------------------------------------------------------------ input transform
// Eight consecutive fp16 values: one 16-byte load when the address allows it (a wave-uniform choice), else eight.
__device__ __forceinline__ h8_t load_h8(const uint16_t* p, bool vec) {
    if (vec) return __builtin_bit_cast(h8_t, ldg(reinterpret_cast<const u32x4_t*>(p)));
    h8_t v;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __builtin_bit_cast(_Float16, ldg(p + j));
    return v;
}

// B fragment (v_mfma_f32_16x16x32_f16 layout: lane L holds column n = L & 15, rows k = 8 (L >> 4) + j) of the 128-point
// Hadamard matrix H[K][N] = (-1)^popcount(K & N) for K in 32 ks + [0, 32), N in 16 nb + [0, 16). popcount(K & N)
// splits into popcount(k & n) (bits 0-3), bit 4 of k with bit 0 of nb, and bits 0-1 of ks with bits 1-2 of nb: the
// fragment is F_{nb & 1} (lane-dependent, bit 4 of k = L >> 5) times the sign S(ks, nb), a compile-time constant.
__device__ __forceinline__ h8_t had_fragment(int lane, int p) {
    const int n = lane & 15, k0 = 8 * (lane >> 4);
    h8_t f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int odd = (__builtin_popcount((unsigned)((k0 + j) & n)) + p * (lane >> 5)) & 1;
        f[j] = odd ? (_Float16)-1.0f : (_Float16)1.0f;
    }
    return f;
}
__host__ __device__ constexpr bool had_sign_neg(int ks, int nb) {
    return (((ks & 1) & ((nb >> 1) & 1)) ^ (((ks >> 1) & 1) & ((nb >> 2) & 1))) != 0;
}

// fp16(H128(fp16(x * s)) / sqrt(128)) of one wave's 16 rows: xv holds the rows' x in A-fragment layout (lane L: row
// L & 15, columns 32 ks + 8 (L >> 4) + j), sv points at s + 8 (L >> 4) (16-byte loads when vs). The results go to the
// wave's LDS tile (16 x 128 fp16) and part[i] gets the sum of the fp16 results of row 4 (L >> 4) + i over this lane's
// 8 columns (the caller reduces over the 16 lanes of a row).
__device__ __forceinline__ void had16_rows(const h8_t (&xv)[4], const h8_t (&sg)[4], const h8_t (&F)[2], int lane,
                                           _Float16 (*tile)[136], float (&part)[4]) {
    const int m = lane & 15, g = lane >> 4;
    h8_t A[4], An[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        A[ks] = xv[ks] * sg[ks];
        An[ks] = -A[ks];
    }
    f4_t acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
        acc[nb] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(had_sign_neg(ks, nb) ? An[ks] : A[ks], F[nb & 1],
                                                             acc[nb], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) part[i] = 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const _Float16 h = (_Float16)(acc[nb][i] * kRsqrt128);
            part[i] += (float)h;
            tile[4 * g + i][16 * nb + m] = h;
        }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// the signs from sv + 32 ks (16-byte loads when vs)
__device__ __forceinline__ void had16_rows(const h8_t (&xv)[4], const uint16_t* sv, bool vs, const h8_t (&F)[2],
                                           int lane, _Float16 (*tile)[136], float (&part)[4]) {
    h8_t sg[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) sg[ks] = load_h8(sv + 32 * ks, vs);
    had16_rows(xv, sg, F, lane, tile, part);
}

// Sum of v over the 16 lanes of a row (lanes with equal L >> 4).
__device__ __forceinline__ float row16_sum(float v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    return v;
}

// One wave per job (16 consecutive pairs of the expert-sorted order, 128-column block kb; jobs row group major, four
// per workgroup): every row's x block times its expert's suh_gate and suh_up, Hadamard / sqrt(128), fp16 (the GEMM
// inputs xh) and their block sums (xsum). Rows are independent here, so a job's rows may belong to several experts
// and no job is empty: the rows' tokens and experts come from the pair arrays in one round trip (no block
// descriptor), then x and the signs in the next. A fragments are fp16(x * suh) (packed fp16 multiplies, one rounding:
// the reference's fp16(x * suh)), the Hadamard is 8 output tiles x 4 k-steps of v_mfma_f32_16x16x32_f16 against the
// two base fragments (fp32 accumulation of exact +-x products), and the sums of the fp16-rounded outputs reduce over
// the 16 lanes of a row.
__global__ __launch_bounds__(256) void pairs_had_kernel(MoeArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 s_out[4][16][136];    // per wave: 16 rows x 128 (+ pad)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nblk = a.H / 128, np = a.M * a.slots;
    const int job = 4 * blockIdx.x + wave, rg = job / nblk, kb = job - rg * nblk, r0 = 16 * rg;
    if (r0 >= np) return;                                    // past the last row group (uniform)
    const int m = lane & 15, g = lane >> 4;
    const int p = r0 + m < np ? r0 + m : np - 1;
    const int tok = a.pair_tok[p], e = a.pair_e[p];
    const bool valid = r0 + m < np && e >= 0;
    const uint32_t vmask = (uint32_t)__builtin_amdgcn_ballot_w64(valid) & 0xFFFFu;   // rows of this job to store
    if (vmask == 0) return;
    const int ec = valid ? e : 0;
    const uint16_t* sgn[2];
    if (a.uniform) {
        sgn[0] = reinterpret_cast<const uint16_t*>(a.tb[1] + (int64_t)ec * a.ts[1]);
        sgn[1] = reinterpret_cast<const uint16_t*>(a.tb[4] + (int64_t)ec * a.ts[4]);
    } else {
        sgn[0] = reinterpret_cast<const uint16_t*>(ldg(a.tables + (int64_t)1 * a.E + ec));
        sgn[1] = reinterpret_cast<const uint16_t*>(ldg(a.tables + (int64_t)4 * a.E + ec));
    }
    const uint16_t* xr = a.x + (int64_t)(valid ? tok : 0) * a.x_ld + kb * 128 + 8 * g;
    const bool vx = ((uintptr_t)a.x & 15) == 0 && (a.x_ld & 7) == 0;
    // x and both projections' signs in one round trip
    h8_t xv[4], sg[2][4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) xv[ks] = load_h8(xr + 32 * ks, vx);
#pragma unroll
    for (int proj = 0; proj < 2; ++proj) {
        const uint16_t* sv = sgn[proj] + kb * 128 + 8 * g;
        const bool vs = __builtin_amdgcn_ballot_w64(((uintptr_t)sv & 15) != 0) == 0;   // every row 16-byte aligned
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) sg[proj][ks] = load_h8(sv + 32 * ks, vs);
    }
    const h8_t F[2] = {had_fragment(lane, 0), had_fragment(lane, 1)};
#pragma unroll
    for (int proj = 0; proj < 2; ++proj) {
        float part[4];
        had16_rows(xv, sg[proj], F, lane, s_out[wave], part);
#pragma unroll
        for (int c = 0; c < 4; ++c) {                   // 16-byte row stores from the tile
            const int u = lane + 64 * c, rr = u >> 4, ch = u & 15;
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&s_out[wave][rr][8 * ch]);
            if ((vmask >> rr) & 1)
                *reinterpret_cast<u32x4_t*>(a.xh + ((size_t)(r0 + rr) * 2 + proj) * a.H + kb * 128 + 8 * ch) = v;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = row16_sum(part[i]);
            if (m == 0 && ((vmask >> (4 * g + i)) & 1)) a.xsum[((size_t)(r0 + 4 * g + i) * 2 + proj) * nblk + kb] = v;
        }
        __builtin_amdgcn_wave_barrier();                // the tile is rewritten by the next projection
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// Block id and column block of this workgroup under the XCD-aware layout (ids round-robin over 8 XCDs).
__device__ __forceinline__ void xcd_map(int nbc, int& blk, int& nb) {
    const int id = blockIdx.x, xcd = id & 7, j = id >> 3;
    const int q = j / nbc;
    blk = 8 * q + xcd;
    nb = j - q * nbc;
}

// ------------------------------------------------------------------------------------------------ pipelined K loop
constexpr int kMfT = 4;                              // tile columns per wave

// Workgroups per CU (= waves per SIMD) the grouped GEMM kernels are compiled for, by row class (1, 2 or 4 row
// groups). The 4-row-group uniform kernels take one more where their registers allow it without spills (168 VGPRs:
// gate|up at K = 1, 2 and 4, down at K <= 4); the 1-row-group kernels run five (96 VGPRs; uniform K up to 4, above
// which they would spill), their epilogue buffer aliasing the pipeline's LDS so that five fit.
#ifndef EXL3_MFMA_OCC1
#define EXL3_MFMA_OCC1 4
#endif
#ifndef EXL3_MFMA_OCC2
#define EXL3_MFMA_OCC2 3
#endif
#ifndef EXL3_MFMA_OCC4
#define EXL3_MFMA_OCC4 2
#endif
#ifndef EXL3_MFMA_OCC1_KMAX
#define EXL3_MFMA_OCC1_KMAX 4
#endif
#define EXL3_MFMA_OCC(RGA) ((RGA) == 1 ? EXL3_MFMA_OCC1 : (RGA) == 2 ? EXL3_MFMA_OCC2 : EXL3_MFMA_OCC4)
#define EXL3_MFMA_GU_OCC(RGA, K) \
    ((RGA) == 4 && ((K) <= 2 || (K) == 4) ? EXL3_MFMA_OCC4 + 1 : (RGA) == 1 && (K) <= EXL3_MFMA_OCC1_KMAX ? 5 \
                                                                   : EXL3_MFMA_OCC(RGA))
#define EXL3_MFMA_DOWN_OCC(RGA, K) \
    ((RGA) == 4 && (K) <= 4 ? EXL3_MFMA_OCC4 + 1 : (RGA) == 1 && (K) <= EXL3_MFMA_OCC1_KMAX ? 5 : EXL3_MFMA_OCC(RGA))
#ifndef EXL3_MIX_OCC1
#define EXL3_MIX_OCC1 5
#endif
#define EXL3_MIX_OCC(RGA) ((RGA) == 1 ? EXL3_MIX_OCC1 : (RGA) == 2 ? 3 : 2)

// 16-byte unit of (row, chunk) in one staged A plane (16 * RGA rows x four 16-byte chunks = 32 k); the chunk is
// swizzled by row so that the 16 rows of a fragment read hit distinct banks.
__device__ __forceinline__ int a_unit(int row, int ch) { return row * 4 + (ch ^ ((row >> 1) & 3)); }

typedef __attribute__((address_space(3))) const uint32_t* lds_cu32_t;
constexpr int kBufferWord3 = 0x00020000;                     // buffer resource word 3 for raw 32-bit loads (gfx9)
// A wave-uniform buffer resource over `p` (loads at offsets below 2^31 bytes; beyond the range they return zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7fffffff, kBufferWord3);
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// One wave accumulates kMfT tile columns over all 32-k steps for RGA row groups. Tile column t of the wave belongs to
// column pair t >> 1 (gate|up: the projection; down: columns c0, c0 + 1 or c0 + 2, c0 + 3), whose two adjacent tiles of
// one tile-row are contiguous in memory.
//   weights: per step the wave's 8 tiles (2 pairs x 2 tile-rows x 2 tiles) come in with ONE coalesced load of K words
//            per lane (16 lanes per 2-tile segment), loaded DW - 1 steps ahead into a register ring, and are staged in a
//            wave-private LDS slot per tile laid out as [w(8K-1), w(0) .. w(8K-1), w(0), w(1), w(2)], so that every
//            lane's fragment window (first word -1 .. 8K - 1, at most 8K + 2 past) is contiguous: no wrap logic, and
//            per-lane scattered loads (64-bit addresses per lane into the texture unit) become LDS reads. For K <= 5
//            the fragments are k-permuted (two funnels of four windows per lane, fragp_finish); K >= 6 keeps the
//            natural k order (frag_finish).
//   A:       staged per step by the whole workgroup: loaded into register slot s % 2 three steps ahead, stored to
//            LDS stage s % 4 two steps ahead, with a barrier after the even steps only (a stage is rewritten two steps
//            after its last read, with a barrier in between, and read at least one barrier after its write); memory-
//            counter waits complete in issue order, so each step issues its A load before its weight load. With
//            k-permuted fragments a row's 4-k units are staged in the order 0 2 1 3 4 6 5 7 (two 8-byte stores per
//            16-byte unit), so that a lane's 16-byte read holds the k of its B fragment. With one row group and one
//            plane read per wave, each wave stages its own plane in a private ring instead (one unit per lane, the
//            loads and LDS writes of the shared ring, whose threads stage its units twice or more) and the loop has no
//            barrier.
template <int K, int NP, int RGA, int NPS = NP, bool PL = false>
struct MfmaPipe {
    static constexpr bool KP = K <= 5;                      // k-permuted fragments
    static constexpr int NW = FragCfg<K>::NW;
    static constexpr int DW = 4;
    static constexpr int TPP = kMfT / NP;
    static constexpr int TS = 8 * K + 4;                     // LDS words per staged tile
    static constexpr int UNITS = NPS * RGA * 64;             // 16-byte A units per stage (NPS staged planes)
    static constexpr bool PRIV = RGA == 1 && NP == 1;        // wave-private A ring
    static constexpr int SU = PRIV ? 64 : UNITS;             // units per stage (of the wave's ring if PRIV)
    static constexpr int CPT = PRIV ? 1 : (UNITS + 255) / 256;   // A units a thread stages per step
    const uint32_t* wsrc;                                    // this lane's K words at step 0
    uint32_t wstep;                                          // words between consecutive steps (two tile-rows)
    int nsteps;
    uint32_t* wl;                                            // the wave's LDS slots [8][TS]
    int wdst, wslot;                                         // this lane's staged words: slot wslot, word wdst
    int w0;                                                  // fragment window origin (ring word, -1 .. 8K - 1)
    uint32_t sh;
    uint32_t fa[2], fsh[2];                                  // k-permuted: LDS byte address of each run's funnel
                                                             // words in slot 0, and its shift
    __amdgpu_buffer_rsrc_t abuf[CPT];                        // this thread's staged A units at step 0: a buffer
    uint32_t aoff[CPT];                                      // the wave shares, and the lane's byte offset in it
    int adst[CPT];                                           // k-permuted: 8-byte units of the low and high halves
    int adst2[CPT];
    u32x4_t* lds;                                            // [4][SU] (per wave if PRIV)
    int lane;
    int apl = 0;                                             // first staged plane this wave reads (NPS > NP)

    __device__ __forceinline__ void load_w(uint32_t (&D)[K], int s) const {
        const uint32_t* p = wsrc + (uint32_t)(s < nsteps ? s : nsteps - 1) * wstep;
#pragma unroll
        for (int i = 0; i < K; ++i) D[i] = ldg_nt(p + WordOrder<K, PL>::word_off(i));
        __builtin_amdgcn_sched_barrier(0);
    }
    __device__ __forceinline__ void stage_w(const uint32_t (&D)[K]) const {
        uint32_t* t = wl + wslot * TS;
#pragma unroll
        for (int i = 0; i < K; ++i) t[1 + wdst + i] = D[i];
        const int q = lane & 7;                              // this lane's eighth of the tile
        if (q == 7) t[0] = D[K - 1];                          // w(8K - 1) in front
#pragma unroll
        for (int u = 0; u < 3; ++u)                          // w(0..2) behind
            if (q == u / K) t[8 * K + 1 + u] = D[u % K];
    }
    __device__ __forceinline__ void compute(int stage, f4_t (&acc)[kMfT][RGA]) const {
        h8_t bf[kMfT];
        if constexpr (KP) {
            uint32_t fw[kMfT][4];
#pragma unroll
            for (int t = 0; t < kMfT; ++t) {
                const int slot = 2 * (2 * (t >> 1) + (lane >> 5)) + (t & 1);
#pragma unroll
                for (int g = 0; g < 2; ++g) {
                    const lds_cu32_t o = (lds_cu32_t)fa[g];
                    fw[t][2 * g] = o[slot * TS];
                    fw[t][2 * g + 1] = o[slot * TS + 1];
                }
            }
#pragma unroll
            for (int t = 0; t < kMfT; ++t) bf[t] = fragp_finish<K>(fw[t], fsh);
        } else {
#pragma unroll
            for (int t = 0; t < kMfT; ++t) {
                const int slot = 2 * (2 * (t >> 1) + (lane >> 5)) + (t & 1);
                const uint32_t* r = wl + slot * TS + 1 + w0;
                uint32_t R[NW];
#pragma unroll
                for (int i = 0; i < NW; ++i) R[i] = r[i];
                bf[t] = frag_finish<K>(R, sh);
            }
        }
        // A fragments per plane, after the B decode (fewer live registers: three waves per SIMD at four row groups)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            h8_t af[RGA];
#pragma unroll
            for (int rg = 0; rg < RGA; ++rg)
                af[rg] = __builtin_bit_cast(
                    h8_t, lds[stage * SU + (PRIV ? 0 : (p + apl) * RGA * 64) + a_unit(16 * rg + (lane & 15), lane >> 4)]);
#pragma unroll
            for (int t = p * TPP; t < (p + 1) * TPP; ++t)
#pragma unroll
                for (int rg = 0; rg < RGA; ++rg)
                    acc[t][rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[rg], bf[t], acc[t][rg], 0, 0, 0);
        }
    }
    // step s, with every ring slot known at compile time (R = s mod 4)
    template <int R>
    __device__ __forceinline__ void step(int s, uint32_t (&W)[DW][K], u32x4_t (&RA)[2][CPT],
                                         f4_t (&acc)[kMfT][RGA]) const {
        load_a(RA[R % 2], s + 3);
        load_w(W[(R + DW - 1) % DW], s + DW - 1);
        stage_w(W[R % DW]);
        compute(R, acc);
        store_a(RA[(R + 1) % 2], (R + 2) % 4);
        if constexpr (!PRIV) {
            if (R % 2 == 0) __syncthreads();
        }
    }
    __device__ __forceinline__ void load_a(u32x4_t (&Ra)[CPT], int s) const {
        const int ss = (s < nsteps ? s : nsteps - 1) * 32;
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            Ra[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(abuf[j], aoff[j], 2 * ss, 0));
        __builtin_amdgcn_sched_barrier(0);
    }
    __device__ __forceinline__ void store_a(const u32x4_t (&Ra)[CPT], int stage) const {
        if constexpr (KP) {
            typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
            u2_t* l2 = reinterpret_cast<u2_t*>(lds) + 2 * stage * SU;
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                const u2_t lo = {Ra[j][0], Ra[j][1]}, hi = {Ra[j][2], Ra[j][3]};
                l2[adst[j]] = lo;
                l2[adst2[j]] = hi;
            }
        } else {
#pragma unroll
            for (int j = 0; j < CPT; ++j) lds[stage * SU + adst[j]] = Ra[j];
        }
    }
    __device__ __forceinline__ void run(f4_t (&acc)[kMfT][RGA]) const {
        uint32_t W[DW][K];
        u32x4_t RA[2][CPT];
        load_a(RA[0], 0);
        load_a(RA[1], 1);
#pragma unroll
        for (int i = 0; i < DW - 1; ++i) load_w(W[i], i);
        store_a(RA[0], 0);
        store_a(RA[1], 1);
        load_a(RA[1], 2);
        __syncthreads();
        int s = 0;
        for (; s + 4 <= nsteps; s += 4) {
            step<0>(s, W, RA, acc);
            step<1>(s + 1, W, RA, acc);
            step<2>(s + 2, W, RA, acc);
            step<3>(s + 3, W, RA, acc);
        }
        if (s < nsteps) step<0>(s, W, RA, acc);
        if (s + 1 < nsteps) step<1>(s + 1, W, RA, acc);
        if (s + 2 < nsteps) step<2>(s + 2, W, RA, acc);
        __syncthreads();                                 // every wave's last LDS read done: callers may reuse it
    }
    // weight set-up: tr = tile-row 0 of the projection, pair_col(pair) = the pair's first tile column (even); tile-rows
    // are tn * 8K words apart. Lane (lane & 15) of a pair segment takes chunk lane & 7 of the pair's tile
    // (lane & 15) >> 3, in the word order PL (WordOrder).
    template <typename F>
    __device__ __forceinline__ void setup_w(int tn, uint32_t* wave_lds, const uint32_t* tr, F pair_col) {
        const int g = lane >> 4, pair = g >> 1, hr = g & 1;
        wsrc = tr + (size_t)hr * tn * (8 * K) +
               WordOrder<K, PL>::chunk_base(pair_col(pair) + ((lane & 15) >> 3), lane & 7);
        wstep = (uint32_t)(2 * tn * 8 * K);
        wl = wave_lds;
        wslot = 2 * g + ((lane & 15) >> 3);
        wdst = (lane & 7) * K;
        if constexpr (KP) {
            int off[2];
            fragp_origin<K>(lane, off, fsh);
#pragma unroll
            for (int g = 0; g < 2; ++g) fa[g] = lds_addr(wl) + 4u * (uint32_t)off[g];
        } else {
            frag_origin<K>(lane, w0, sh);
        }
    }
    // staging set-up: unit u = (tid + 256 j) mod UNITS (UNITS < 256: several threads stage the same unit, writing
    // the same value, so that the loads and stores stay unconditional: a branch around them would make the compiler
    // drain every outstanding load, the weight prefetch included) of plane p = u / (RGA * 64): row (u % (RGA * 64)) / 4
    // (clamped to the block's last row), chunk u % 4, from row pointer rowptr(p, row) (k offset 0). A wave's 64 units
    // lie in one plane (UNITS and RGA * 64 are multiples of 64), so the loads are buffer loads from the plane's row 0
    // (a wave-uniform resource) at a 32-bit lane offset plus the step's scalar offset: no address arithmetic per step.
    template <typename F>
    __device__ __forceinline__ void setup_a(int cnt, F rowptr) {
        const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        if constexpr (PRIV) lds += wv * 4 * SU;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int u0 = PRIV ? apl * 64 : (64 * wv + 256 * j) % UNITS, u = u0 + (threadIdx.x & 63);
            const int p = u0 / (RGA * 64), rem = u - p * RGA * 64, row = rem >> 2, ch = rem & 3;
            const int pd = PRIV ? 0 : p;                     // the unit's plane in the stage
            const _Float16* b = rowptr(p, 0);
            abuf[j] = buffer_rsrc(b);
            aoff[j] = (uint32_t)(2 * (rowptr(p, row < cnt ? row : cnt - 1) + 8 * ch - b));
            if constexpr (KP) {                              // 4-k units 2 ch, 2 ch + 1 -> 16-byte units
                adst[j] = 2 * (pd * RGA * 64 + a_unit(row, ch & 2)) + (ch & 1);       // (ch & 2) and (ch & 2) + 1,
                adst2[j] = 2 * (pd * RGA * 64 + a_unit(row, (ch & 2) + 1)) + (ch & 1); // half ch & 1
            } else {
                adst[j] = pd * RGA * 64 + a_unit(row, ch);
            }
        }
    }
};

// ------------------------------------------------------------------------------------------------ gate | up
template <int RGA>
__device__ __forceinline__ void gateup_epilogue(const MoeArgs& a, const ItemDesc* d, int nb, int cnt,
                                                const f4_t (&acc)[kMfT][RGA], float* C, const float* rsum);
template <int RGA>
__device__ __forceinline__ void down_epilogue(const MoeArgs& a, const ItemDesc* d, int nb, int cnt,
                                              const f4_t (&acc)[kMfT][RGA], float* C, const float* rsum, int* s_comb);

template <int K, int RGA, bool PL>
__device__ __forceinline__ void gateup_mfma_body(const MoeArgs& a, const ItemDesc* d, int nb, int cnt, u32x4_t* stage,
                                                 uint32_t* wlds, float* C, float* rsum) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p0 = d->p0;
    const int tn = a.gu_tn;
    const int pw = wave >> 1;                              // this wave's projection (gate, up), its 4 tile columns
    const uint32_t* trp = reinterpret_cast<const uint32_t*>(d->tab[3 * pw]);
    const int ct0 = nb * 8 + 4 * (wave & 1);
    MfmaPipe<K, 1, RGA, 2, PL> L;
    L.nsteps = a.H / 32;
    L.lds = stage;
    L.lane = lane;
    L.apl = pw;
    L.setup_w(tn, wlds + wave * 8 * (8 * K + 4), trp, [&](int pair) { return ct0 + 2 * pair; });
    L.setup_a(cnt, [&](int p, int row) { return a.xh + ((size_t)(p0 + row) * 2 + p) * a.H; });
    f4_t acc[kMfT][RGA];
#pragma unroll
    for (int t = 0; t < kMfT; ++t)
#pragma unroll
        for (int rg = 0; rg < RGA; ++rg) acc[t][rg] = f4_t{0.f, 0.f, 0.f, 0.f};
    L.run(acc);
    gateup_epilogue<RGA>(a, d, nb, cnt, acc, C, rsum);
}

// Affine, Hadamard * svh, act(g, u) * suh_d, Hadamard of the workgroup's 128 columns per 16-row group -> abuf (fp16)
// and its block sums (the down GEMM's affine term).
template <int RGA>
__device__ __forceinline__ void gateup_epilogue(const MoeArgs& a, const ItemDesc* d, int nb, int cnt,
                                                const f4_t (&acc)[kMfT][RGA], float* C, const float* rsum) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p0 = d->p0;
    const uint16_t* svg = reinterpret_cast<const uint16_t*>(d->tab[2]) + nb * 128;
    const uint16_t* svu = reinterpret_cast<const uint16_t*>(d->tab[5]) + nb * 128;
    const uint16_t* sud = reinterpret_cast<const uint16_t*>(d->tab[7]) + nb * 128;
    const float sg0 = h2f(ldg(svg + lane)), sg1 = h2f(ldg(svg + lane + 64));
    const float su0 = h2f(ldg(svu + lane)), su1 = h2f(ldg(svu + lane + 64));
    const float sd0 = h2f(ldg(sud + lane)), sd1 = h2f(ldg(sud + lane + 64));
    const int nbI = a.I / 128;
#pragma unroll
    for (int rg = 0; rg < RGA; ++rg) {
        // this row group's gate / up columns of the whole workgroup -> C[2][16][128]; wave w holds projection w >> 1,
        // tile columns 4 (w & 1) .. + 3 of the block
#pragma unroll
        for (int t = 0; t < kMfT; ++t) {
            const int p = wave >> 1, col = (4 * (wave & 1) + t) * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) C[(p * 16 + 4 * (lane >> 4) + i) * 128 + col] = acc[t][rg][i];
        }
        __syncthreads();
        for (int j = 0; j < 4; ++j) {
            const int ml = 4 * wave + j, m = 16 * rg + ml;
            if (m >= cnt) break;
            const float sg = kMul1C2 * rsum[m], su = kMul1C2 * rsum[64 + m];
            float g0 = kMul1C1 * C[ml * 128 + lane] + sg, g1 = kMul1C1 * C[ml * 128 + lane + 64] + sg;
            float u0 = kMul1C1 * C[(16 + ml) * 128 + lane] + su, u1 = kMul1C1 * C[(16 + ml) * 128 + lane + 64] + su;
            fwht128_wave(g0, g1, lane);
            fwht128_wave(u0, u1, lane);
            g0 = (float)(_Float16)(g0 * kRsqrt128 * sg0);
            g1 = (float)(_Float16)(g1 * kRsqrt128 * sg1);
            u0 = (float)(_Float16)(u0 * kRsqrt128 * su0);
            u1 = (float)(_Float16)(u1 * kRsqrt128 * su1);
            float a0 = (float)(_Float16)act_mul_dev(g0, u0, a.act, a.limit);
            float a1 = (float)(_Float16)act_mul_dev(g1, u1, a.act, a.limit);
            a0 = (float)(_Float16)(a0 * sd0);
            a1 = (float)(_Float16)(a1 * sd1);
            fwht128_wave(a0, a1, lane);
            const _Float16 h0 = (_Float16)(a0 * kRsqrt128), h1 = (_Float16)(a1 * kRsqrt128);
            uint16_t* dst = a.abuf + (size_t)(p0 + m) * a.I + nb * 128;
            dst[lane] = __builtin_bit_cast(uint16_t, h0);
            dst[lane + 64] = __builtin_bit_cast(uint16_t, h1);
            const float bs = wave_sum_f32((float)h0 + (float)h1);
            if (lane == 0) a.asum[(size_t)(p0 + m) * nbI + nb] = bs;
        }
        __syncthreads();
    }
}

// sum over b < n of q[b] (n >= 1), in order, with the loads issued 16 at a time (unconditionally: indices clamped to
// n - 1, so no branch splits a batch into separate round trips)
__device__ __forceinline__ float sum_ordered(const float* q, int n) {
    float v = 0.f;
    for (int b0 = 0; b0 < n; b0 += 16) {
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) t[i] = ldg(q + (b0 + i < n ? b0 + i : n - 1));
#pragma unroll
        for (int i = 0; i < 16; ++i) v += b0 + i < n ? t[i] : 0.f;
    }
    return v;
}

// One instance per row class (RGA row groups of 16): workgroup (list index, column block); indices past the class's
// block count exit at once.
template <int K, int RGA, bool PL = false>
__global__ __launch_bounds__(256, EXL3_MFMA_GU_OCC(RGA, K)) void gateup_mfma_kernel(MoeArgs a) {
    constexpr int CL = RGA == 1 ? 0 : RGA == 2 ? 1 : 2;
    // A stages [4][2 planes][16 RGA rows x 4 units] (or per wave [4][16 rows x 4 units]) and per wave 8 staged tiles;
    // the epilogue's C reuses them (dead once the pipeline has drained)
    constexpr int kStage = 4 * (RGA == 1 ? 4 : 2 * RGA) * 64 * 16, kW = 4 * 8 * (8 * K + 4) * 4, kC = 2 * 16 * 128 * 4;
    __shared__ __attribute__((aligned(16))) char smem[kStage + kW > kC ? kStage + kW : kC];
    u32x4_t* stage = reinterpret_cast<u32x4_t*>(smem);
    uint32_t* wlds = reinterpret_cast<uint32_t*>(smem + kStage);
    float* C = reinterpret_cast<float*>(smem);
    __shared__ float rsum[2 * 64];
    const int nbI = a.I / 128;
    int idx, nb;
    xcd_map(nbI, idx, nb);
    if (idx >= a.cls_cnt[CL]) return;
    const ItemDesc* d = a.blocks + a.cls_list[CL * a.max_blocks + idx];
    const int cnt = d->cnt;
    // row sums of the block's A rows (block sums in order)
    const int nblk = a.H / 128;
    for (int i = threadIdx.x; i < 2 * 64; i += 256) {
        const int p = i >> 6, m = i & 63;
        rsum[i] = m < cnt ? sum_ordered(a.xsum + ((size_t)(d->p0 + m) * 2 + p) * nblk, nblk) : 0.f;
    }
    __syncthreads();
    gateup_mfma_body<K, RGA, PL>(a, d, nb, cnt, stage, wlds, C, rsum);
}

// ------------------------------------------------------------------------------------------------ down
// 256 output columns per workgroup (two Hadamard blocks): wave w owns tile columns 4w .. 4w + 3.
template <int K, int RGA, bool PL>
__device__ __forceinline__ void down_mfma_body(const MoeArgs& a, const ItemDesc* d, int nb, int cnt, u32x4_t* stage,
                                               uint32_t* wlds, float* C, float* rsum, int* s_comb) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p0 = d->p0;
    const int tn = a.H / 16;
    const uint32_t* trd = reinterpret_cast<const uint32_t*>(d->tab[6]);
    MfmaPipe<K, 1, RGA, 1, PL> L;
    L.nsteps = a.I / 32;
    L.lds = stage;
    L.lane = lane;
    L.setup_w(tn, wlds + wave * 8 * (8 * K + 4), trd, [&](int pair) {
        const int ct = nb * 16 + 4 * wave + 2 * pair;
        return ct < tn ? ct : tn - 2;                  // a last half block: in-bounds loads, results unused
    });
    L.setup_a(cnt, [&](int, int row) { return reinterpret_cast<const _Float16*>(a.abuf) + (size_t)(p0 + row) * a.I; });
    f4_t acc[kMfT][RGA];
#pragma unroll
    for (int t = 0; t < kMfT; ++t)
#pragma unroll
        for (int rg = 0; rg < RGA; ++rg) acc[t][rg] = f4_t{0.f, 0.f, 0.f, 0.f};
    L.run(acc);
    down_epilogue<RGA>(a, d, nb, cnt, acc, C, rsum, s_comb);
}

// Affine, Hadamard * svh_d * w of the workgroup's 256 columns per 16-row group -> y rows, then the combine.
template <int RGA>
__device__ __forceinline__ void down_epilogue(const MoeArgs& a, const ItemDesc* d, int nb, int cnt,
                                              const f4_t (&acc)[kMfT][RGA], float* C, const float* rsum, int* s_comb) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p0 = d->p0;
    const int nbH = a.H / 128;
    const int nhalf = 2 * nb + 1 < nbH ? 2 : 1;
    const uint16_t* svd = reinterpret_cast<const uint16_t*>(d->tab[8]) + nb * 256;
    float sd[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int hh = h < nhalf ? h : 0;                // unconditional load, unused past nhalf
        sd[h][0] = h2f(ldg(svd + 128 * hh + lane));
        sd[h][1] = h2f(ldg(svd + 128 * hh + lane + 64));
    }
    // row weights of this wave's rows 16 rg + 4 wave + r, all loaded before the first is needed
    float wr[RGA][4];
#pragma unroll
    for (int rg = 0; rg < RGA; ++rg)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 16 * rg + 4 * wave + r;
            wr[rg][r] = a.pair_w[p0 + (m < cnt ? m : cnt - 1)];
        }
#pragma unroll
    for (int rg = 0; rg < RGA; ++rg) {
#pragma unroll
        for (int t = 0; t < kMfT; ++t) {
            const int col = (4 * wave + t) * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) C[(4 * (lane >> 4) + i) * 256 + col] = acc[t][rg][i];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 8; ++j) {                 // (row, half) pairs of this wave
            const int ml = 4 * wave + (j >> 1), h = j & 1, m = 16 * rg + ml;
            if (m >= cnt || h >= nhalf) continue;
            const float sx = kMul1C2 * rsum[m];
            float v0 = kMul1C1 * C[ml * 256 + 128 * h + lane] + sx, v1 = kMul1C1 * C[ml * 256 + 128 * h + lane + 64] + sx;
            fwht128_wave(v0, v1, lane);
            const float w = wr[rg][j >> 1];
            float* dst = a.y + (size_t)(p0 + m) * a.H + nb * 256 + 128 * h;
            splitk_store(dst + lane, v0 * kRsqrt128 * sd[h][0] * w);
            splitk_store(dst + lane + 64, v1 * kRsqrt128 * sd[h][1] * w);
        }
        __syncthreads();
    }
    // combine: count rows into their tokens per 128-column block, finish tokens whose slots are all in
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int i = threadIdx.x; i < 2 * cnt; i += 256) {
        const int m = i >> 1, h = i & 1;
        int r = -1;
        if (h < nhalf) {
            const int t = a.pair_tok[p0 + m];
            const int old = __hip_atomic_fetch_add(&a.cnt_tok[(size_t)t * nbH + 2 * nb + h], 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
            r = (old == a.tok_nvalid[t] - 1) ? t : -1;
        }
        s_comb[i] = r;
    }
    __syncthreads();
    for (int i = wave; i < 2 * cnt; i += 4)
        if (s_comb[i] >= 0) combine_token(a, s_comb[i], 2 * nb + (i & 1), lane);
}

template <int K, int RGA, bool PL = false>
__global__ __launch_bounds__(256, EXL3_MFMA_DOWN_OCC(RGA, K)) void down_mfma_kernel(MoeArgs a) {
    constexpr int CL = RGA == 1 ? 0 : RGA == 2 ? 1 : 2;
    // A stages [4][16 RGA rows x 4 units] (per wave at one row group) and per wave 8 staged tiles; C aliases, as above
    constexpr int kStage = 4 * (RGA == 1 ? 4 : RGA) * 64 * 16, kW = 4 * 8 * (8 * K + 4) * 4, kC = 16 * 256 * 4;
    __shared__ __attribute__((aligned(16))) char smem[kStage + kW > kC ? kStage + kW : kC];
    u32x4_t* stage = reinterpret_cast<u32x4_t*>(smem);
    uint32_t* wlds = reinterpret_cast<uint32_t*>(smem + kStage);
    float* C = reinterpret_cast<float*>(smem);
    __shared__ float rsum[64];
    __shared__ int s_comb[2 * 64];
    const int nbH2 = (a.H / 128 + 1) / 2;
    int idx, nb;
    xcd_map(nbH2, idx, nb);
    if (idx >= a.cls_cnt[CL]) return;
    const ItemDesc* d = a.blocks + a.cls_list[CL * a.max_blocks + idx];
    const int cnt = d->cnt;
    const int nbI = a.I / 128;
    for (int m = threadIdx.x; m < 64; m += 256)
        rsum[m] = m < cnt ? sum_ordered(a.asum + (size_t)(d->p0 + m) * nbI, nbI) : 0.f;
    __syncthreads();
    down_mfma_body<K, RGA, PL>(a, d, nb, cnt, stage, wlds, C, rsum, s_comb);
}

// ------------------------------------------------------------------------------------------------ per-tile K
// Per-tile bitrate (K = 0: tile i of a projection holds 8 kmap[i] words at woff[i]). Each lane decodes 4 k of one
// tile, so the 64 lanes of a wave always share one tile and its K is wave-uniform. Fragment layout (16x16x16): B[k][n]
// lane L holds n = L & 15, k = 4 (L >> 4) + j, j < 4; A[m][k] lane L holds m = L & 15, same k; D[m][n] n = L & 15,
// m = 4 (L >> 4) + i (the tile rows behind the k slots are permuted, see decode4p). Steps whose tiles are all K <= 2
// join the two tile-rows of a column in one 16x16x32 MFMA (8 k per lane: 4 of each tile).
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
constexpr int kMixKMax = 8;
constexpr int kMixTS = 8 * kMixKMax + 4;                    // LDS words per staged tile: 3 pad, w(8K - 1), 64 words

// k-permuted fragments. An MFMA sums over k, so B and A may list a tile-row's 16 k in any common order. In the order
// used here lane L's four k slots are tile rows 2g, 2g + 1, 2g + 8, 2g + 9 (g = L >> 4) of column n = L & 15: the
// positions t0 .. t0 + 3, t0 = 32 (n & 7) + 4 (n >> 3) + 8 g, four consecutive windows (row 8 ((t >> 1) & 1) +
// 2 ((t >> 3) & 3) + (t & 1), column (t >> 5) + 8 ((t >> 2) & 1)). Their bits [(t0 + 1) K - 16, (t0 + 4) K) fit one
// funnel-shifted word for K <= 5: window b sits at bit 16 - b K of it.
// Seen from 3 words into a staged slot (v = slot + 3): v[0] = ring word 8K - 1, v[1 + w] = ring word w. A funnel whose
// first bit is ring bit `start` (>= -16) reads v[(start + 31) >> 5] and the next word, shifted by
// 31 - ((start + 31) & 31). The windows of positions t <= 255 end inside the ring, so a funnel's second word may lie
// past it (any value: none of its bits is used).
__device__ __forceinline__ h4_t decode4p(uint32_t F, int K) {
    const uint32_t w0 = F >> 16;
    const uint32_t w1 = __builtin_amdgcn_ubfe(F, 16 - K, 16);
    const uint32_t w2 = __builtin_amdgcn_ubfe(F, 16 - 2 * K, 16);
    const uint32_t w3 = __builtin_amdgcn_ubfe(F, 16 - 3 * K, 16);
    typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
    const u2_t v = {__builtin_bit_cast(uint32_t, mul1_pair_raw(w0, w1)),
                    __builtin_bit_cast(uint32_t, mul1_pair_raw(w2, w3))};
    return __builtin_bit_cast(h4_t, v);
}

// K = 2 (k2) or 1: decode4p with the window offsets as constants picked by a wave-uniform flag.
__device__ __forceinline__ h4_t decode4p12(uint32_t F, bool k2) {
    const uint32_t w0 = F >> 16;
    const uint32_t w1 = __builtin_amdgcn_ubfe(F, k2 ? 14 : 15, 16);
    const uint32_t w2 = __builtin_amdgcn_ubfe(F, k2 ? 12 : 14, 16);
    const uint32_t w3 = __builtin_amdgcn_ubfe(F, k2 ? 10 : 13, 16);
    typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
    const u2_t v = {__builtin_bit_cast(uint32_t, mul1_pair_raw(w0, w1)),
                    __builtin_bit_cast(uint32_t, mul1_pair_raw(w2, w3))};
    return __builtin_bit_cast(h4_t, v);
}

// Any K (1 .. 8): the funnel origin from the lane's t0 + 1 at run time, and a second funnel for windows 2 and 3.
__device__ __forceinline__ h4_t decode4p_rt(const uint32_t* slot, int K, uint32_t t0p1) {   // slot: v above
    const uint32_t ta = t0p1 * (uint32_t)K + 15u, tb = ta + 2u * (uint32_t)K;     // start + 31 of windows 0 and 2
    const uint32_t* pa = slot + (ta >> 5);
    const uint32_t* pb = slot + (tb >> 5);
    const uint32_t Fa = __builtin_amdgcn_alignbit(pa[0], pa[1], ~ta);
    const uint32_t Fb = __builtin_amdgcn_alignbit(pb[0], pb[1], ~tb);
    typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
    const u2_t v = {__builtin_bit_cast(uint32_t, mul1_pair_raw(Fa >> 16, __builtin_amdgcn_ubfe(Fa, 16 - K, 16))),
                    __builtin_bit_cast(uint32_t, mul1_pair_raw(Fb >> 16, __builtin_amdgcn_ubfe(Fb, 16 - K, 16)))};
    return __builtin_bit_cast(h4_t, v);
}

// One wave, kMfT tile columns (column pair t >> 1: gate|up projection, or down columns c0 + 2 (t >> 1)), RGA row
// groups, 32 k per step = two tile-rows. Per step the wave's 8 tiles (slot 2t + tile-row half) are fetched by 8 lanes
// each (lane i of a tile: words min(4i, 8K - 4) .. + 3, a 16-byte load inside the tile, and for K >= 5 words
// min(32 + 4i, 8K - 4) .. + 3 at staging time) after their (kmap, woff) one step earlier, and staged in a wave-private
// LDS slot per tile at lane-fixed positions: ring word w at slot[4 + w] (lanes past the tile's end leave copies of its
// last words behind it), the last word w(8K - 1) again at slot[3] (written by lane 7, whose last load always ends the
// tile), so that a funnel starting before the ring reads it. The step's 8 bitrates come from its lanes' kmap bytes (wave ballots): a step
// whose tiles are all K <= 2 stages compactly (slot stride kMixTSF, the first load only) and decodes with per-lane funnel origins
// and shifts precomputed for K = 1 and 2 (one select each per tile); other steps stage at stride kMixTS and decode
// with the tile's K at run time. Rings of 4 (first tile words DW - 1 = 2 steps ahead, (K, woff) DW = 3 steps ahead) make
// the loop a 4-step unroll; the step count (H / 32 or I / 32, H and I multiples of 128) is a multiple of 4. A is staged
// as in MfmaPipe (four LDS stages written two steps ahead, a barrier every second step), but from a register ring of
// two: loaded three steps ahead, stored one step later (the 1-row-group kernels fit five waves per SIMD that way); with
// one row group each wave stages its own plane in a private ring and the loop has no barrier.
constexpr int kMixTSF = 20;                                 // compact slot: 3 pad, w(8K - 1), 16 words (K <= 2)


template <int NPS, int RGA>
struct MfmaPipeMix {
    static constexpr int DW = 3;
    static constexpr int UNITS = NPS * RGA * 64;             // NPS staged A planes; a wave reads plane apl
    // One row group: each wave stages its own plane (64 units, one per lane) in a private ring, so the loop needs no
    // barrier; the loads and LDS writes are those of the shared ring, whose 256 threads stage its units twice or more.
    static constexpr bool PRIV = RGA == 1;
    static constexpr int SU = PRIV ? 64 : UNITS;             // 16-byte units per stage (of the wave's ring if PRIV)
    static constexpr int CPT = PRIV ? 1 : (UNITS + 255) / 256;
    static constexpr int kNT = 2;                            // buffer-load cache policy: nontemporal
    __amdgpu_buffer_rsrc_t wrs, krs, ors;                    // the wave's projection: words, kmap, woff
    int col[2];                                              // per column pair: its first tile column (even)
    int tn, nsteps;
    int apl = 0;
    uint32_t* wl;                                            // the wave's LDS slots [8][kMixTS]
    uint32_t ktile;                                          // this lane's tile entry at step 0 (its slot's tile)
    uint32_t t0p1;                                           // t0 + 1 of the lane's k-permuted positions
    uint32_t fa1, fa2;                                       // fast path: LDS byte address of the lane's funnel
    uint32_t sh1, sh2;                                       // word in compact slot 0 at K = 1 and 2, and the
                                                             // funnel shifts
    __amdgpu_buffer_rsrc_t abuf[CPT];                        // as in MfmaPipe
    uint32_t aoff[CPT];
    int adst[CPT];
    u32x4_t* lds;
    int lane;

    // The step's tile bitrates come from the kmap bytes its lanes loaded (lane 8 sl + i holds slot sl's K), as two
    // wave ballots: `big` (some K > 2: the run-time decode, which reads each K with v_readlane) and `two` (bit 8 sl:
    // slot sl has K = 2, else 1 on the fast path). Scalar loads of the kmap are avoided on purpose: they share the
    // LDS wait counter and may return out of order, so every LDS wait after one would wait for it too.
    __device__ __forceinline__ void load_meta(int (&M)[2], int s) const {
        const int off = (s < nsteps ? s : nsteps - 1) * 2 * tn;
        M[0] = __builtin_amdgcn_raw_buffer_load_b8(krs, ktile, off, 0);
        M[1] = (int)__builtin_amdgcn_raw_buffer_load_b32(ors, 4 * ktile, 4 * off, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
    __device__ __forceinline__ u32x4_t load_words(const int (&M)[2], uint32_t first) const {
        const uint32_t e = 8u * (uint32_t)M[0] - 4u;
        return __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wrs, 4u * ((uint32_t)M[1] + (first < e ? first : e)), 0, kNT));
    }
    // the lane's first 16 bytes of its tile: words min(4i, 8K - 4) .. + 3 (all of the tile for K <= 4)
    __device__ __forceinline__ void load_w(u32x4_t& D, const int (&M)[2]) const {
        D = load_words(M, 4u * (uint32_t)(lane & 7));
        __builtin_amdgcn_sched_barrier(0);
    }
    // Stage the step's tiles (M: this lane's (K, woff)). Lane 7's last loaded word ends its tile, so it writes the
    // wrap word. Tiles of K >= 5 (words 32 .. 8K - 1) take a second load here, on the spot: such steps are rare, and
    // keeping a second register ring for them would cost every step occupancy.
    __device__ __forceinline__ void stage_w(const u32x4_t& D, const int (&M)[2], bool fast, bool big) const {
        const int sl = lane >> 3, i = lane & 7;
        if (fast) {
            uint32_t* t = wl + sl * kMixTSF;
            if (i < 4) *reinterpret_cast<u32x4_t*>(t + 4 + 4 * i) = D;
            if (i == 7) t[3] = D[3];
        } else {
            uint32_t* t = wl + sl * kMixTS;
            *reinterpret_cast<u32x4_t*>(t + 4 + 4 * i) = D;
            if (big) {
                const u32x4_t D1 = load_words(M, 32u + 4u * (uint32_t)i);
                *reinterpret_cast<u32x4_t*>(t + 36 + 4 * i) = D1;
                if (i == 7) t[3] = D1[3];
            } else if (i == 7) {
                t[3] = D[3];
            }
        }
    }
    // A fragments (plane apl) of tile-row half sr in the k-permuted order: k 2g, 2g + 1 from chunk 2 sr, 2g + 8, 2g + 9
    // from chunk 2 sr + 1 (4 bytes at 4g in each unit)
    __device__ __forceinline__ void load_af(int stage, int sr, h4_t (&af)[RGA]) const {
        const int g = lane >> 4;
#pragma unroll
        for (int rg = 0; rg < RGA; ++rg) {
            const u32x4_t* base = lds + stage * SU + (PRIV ? 0 : apl * RGA * 64);
            const int row = 16 * rg + (lane & 15);
            typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
            const u2_t v = {reinterpret_cast<const uint32_t*>(base + a_unit(row, 2 * sr))[g],
                            reinterpret_cast<const uint32_t*>(base + a_unit(row, 2 * sr + 1))[g]};
            af[rg] = __builtin_bit_cast(h4_t, v);
        }
    }
    // slot sl = 2 t + sr holds tile column t (pair t >> 1, parity t & 1) of tile-row half sr; m0 = this lane's K
    __device__ __forceinline__ void compute(int stage, f4_t (&acc)[kMfT][RGA], int m0, uint64_t two, bool fast) const {
        if (fast) {
            // both tile-row halves in one 16x16x32 MFMA per tile column: lane group g's eight k slots are its four of
            // half 0 then its four of half 1, in A and B alike
            h4_t af[2][RGA];
            load_af(stage, 0, af[0]);
            load_af(stage, 1, af[1]);
#pragma unroll
            for (int t = 0; t < kMfT; ++t) {
                uint32_t whi[2], wlo[2];                         // the two tiles' funnel words, both reads issued first
#pragma unroll
                for (int sr = 0; sr < 2; ++sr) {
                    const int sl = 2 * t + sr;
                    const bool k2 = (two >> (8 * sl)) & 1;       // wave-uniform select
                    const lds_cu32_t o = (lds_cu32_t)(k2 ? fa2 : fa1);
                    whi[sr] = o[sl * kMixTSF];
                    wlo[sr] = o[sl * kMixTSF + 1];
                }
                h4_t bf[2];
#pragma unroll
                for (int sr = 0; sr < 2; ++sr) {
                    const bool k2 = (two >> (8 * (2 * t + sr))) & 1;
                    bf[sr] = decode4p12(__builtin_amdgcn_alignbit(whi[sr], wlo[sr], k2 ? sh2 : sh1), k2);
                }
                const h8_t b8 = __builtin_shufflevector(bf[0], bf[1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int rg = 0; rg < RGA; ++rg) {
                    const h8_t a8 = __builtin_shufflevector(af[0][rg], af[1][rg], 0, 1, 2, 3, 4, 5, 6, 7);
                    acc[t][rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8, b8, acc[t][rg], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int sr = 0; sr < 2; ++sr) {
                h4_t af[RGA];
                load_af(stage, sr, af);
#pragma unroll
                for (int t = 0; t < kMfT; ++t) {
                    const int sl = 2 * t + sr;
                    const h4_t bf = decode4p_rt(wl + sl * kMixTS + 3, __builtin_amdgcn_readlane(m0, 8 * sl), t0p1);
#pragma unroll
                    for (int rg = 0; rg < RGA; ++rg)
                        acc[t][rg] = __builtin_amdgcn_mfma_f32_16x16x16f16(af[rg], bf, acc[t][rg], 0, 0, 0);
                }
            }
        }
    }
    __device__ __forceinline__ void load_a(u32x4_t (&Ra)[CPT], int s) const {
        const int ss = (s < nsteps ? s : nsteps - 1) * 32;
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            Ra[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(abuf[j], aoff[j], 2 * ss, 0));
        __builtin_amdgcn_sched_barrier(0);
    }
    __device__ __forceinline__ void store_a(const u32x4_t (&Ra)[CPT], int stage) const {
#pragma unroll
        for (int j = 0; j < CPT; ++j) lds[stage * SU + adst[j]] = Ra[j];
    }
    // step s, R = s mod 4
    template <int R>
    __device__ __forceinline__ void step(int s, u32x4_t (&W)[4], int (&M)[4][2], u32x4_t (&RA)[2][CPT],
                                         f4_t (&acc)[kMfT][RGA]) const {
        load_a(RA[R % 2], s + 3);
        load_meta(M[(R + DW) % 4], s + DW);
        load_w(W[(R + DW - 1) % 4], M[(R + DW - 1) % 4]);
        const int m0 = M[R][0];
        const uint64_t two = __builtin_amdgcn_ballot_w64(m0 == 2);
        const bool fast = __builtin_amdgcn_ballot_w64(m0 > 2) == 0;
        stage_w(W[R], M[R], fast, !fast && __builtin_amdgcn_ballot_w64(m0 > 4) != 0);
        compute(R, acc, m0, two, fast);
        store_a(RA[(R + 1) % 2], (R + 2) % 4);
        if constexpr (!PRIV) {
            if (R % 2 == 0) __syncthreads();
        }
    }
    __device__ __forceinline__ void run(f4_t (&acc)[kMfT][RGA]) const {
        u32x4_t W[4];
        int M[4][2];
        u32x4_t RA[2][CPT];
#pragma unroll
        for (int i = 0; i < DW; ++i) load_meta(M[i], i);
        load_a(RA[0], 0);
        load_a(RA[1], 1);
#pragma unroll
        for (int i = 0; i < DW - 1; ++i) load_w(W[i], M[i]);
        store_a(RA[0], 0);
        store_a(RA[1], 1);
        load_a(RA[1], 2);
        __syncthreads();
        for (int s = 0; s < nsteps; s += 4) {
            step<0>(s, W, M, RA, acc);
            step<1>(s + 1, W, M, RA, acc);
            step<2>(s + 2, W, M, RA, acc);
            step<3>(s + 3, W, M, RA, acc);
        }
        __syncthreads();                                 // every wave's last LDS read done: callers may reuse it
    }
    // After col / tn / wl / lane are set: the lane's tile entry and fast-path origins, and the A staging of `cnt` rows
    // (rowptr(plane, row) -> that row's first element)
    template <typename F>
    __device__ __forceinline__ void setup_a(int cnt, F rowptr) {
        const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        if constexpr (PRIV) {                                // the wave's ring: lds + 4 stages * 64 units per wave
            lds += wv * 4 * SU;
            const int row = lane >> 2, ch = lane & 3;
            const _Float16* b = rowptr(apl, 0);
            abuf[0] = buffer_rsrc(b);
            aoff[0] = (uint32_t)(2 * (rowptr(apl, row < cnt ? row : cnt - 1) + 8 * ch - b));
            adst[0] = a_unit(row, ch);
        } else {
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                const int u0 = (64 * wv + 256 * j) % UNITS, u = u0 + (threadIdx.x & 63);
                const int p = u0 / (RGA * 64), rem = u - p * RGA * 64, row = rem >> 2, ch = rem & 3;
                const _Float16* b = rowptr(p, 0);
                abuf[j] = buffer_rsrc(b);
                aoff[j] = (uint32_t)(2 * (rowptr(p, row < cnt ? row : cnt - 1) + 8 * ch - b));
                adst[j] = p * RGA * 64 + a_unit(row, ch);
            }
        }
        const int sl = lane >> 3, t = sl >> 1, hr = sl & 1, pr = t >> 1;
        ktile = (uint32_t)(hr * tn + (pr ? col[1] : col[0]) + (t & 1));
        const int n = lane & 15, g = lane >> 4;
        t0p1 = (uint32_t)(32 * (n & 7) + 4 * (n >> 3) + 8 * g + 1);
        const uint32_t ta1 = t0p1 + 15u, ta2 = 2u * t0p1 + 15u;           // start + 31 at K = 1, 2
        fa1 = lds_addr(wl) + 4u * (3u + (ta1 >> 5));
        fa2 = lds_addr(wl) + 4u * (3u + (ta2 >> 5));
        sh1 = ~ta1 & 31u;
        sh2 = ~ta2 & 31u;
    }
};

template <int RGA>
__device__ __forceinline__ void gateup_mix_body(const MoeArgs& a, const ItemDesc* d, int nb, int cnt, u32x4_t* stage,
                                                uint32_t* wlds, float* C, float* rsum) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p0 = d->p0;
    MfmaPipeMix<2, RGA> L;
    L.tn = a.I / 16;
    L.nsteps = a.H / 32;
    L.lds = stage;
    L.lane = lane;
    L.wl = wlds + wave * 8 * kMixTS;
    const int pw = wave >> 1;                              // this wave's projection (gate, up), its 4 tile columns
    L.apl = pw;
    L.wrs = buffer_rsrc(reinterpret_cast<const void*>(d->tab[3 * pw]));
    L.krs = buffer_rsrc(reinterpret_cast<const void*>(d->km[2 * pw]));
    L.ors = buffer_rsrc(reinterpret_cast<const void*>(d->km[2 * pw + 1]));
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) L.col[pr] = nb * 8 + 4 * (wave & 1) + 2 * pr;
    L.setup_a(cnt, [&](int p, int row) { return a.xh + ((size_t)(p0 + row) * 2 + p) * a.H; });
    f4_t acc[kMfT][RGA];
#pragma unroll
    for (int t = 0; t < kMfT; ++t)
#pragma unroll
        for (int rg = 0; rg < RGA; ++rg) acc[t][rg] = f4_t{0.f, 0.f, 0.f, 0.f};
    L.run(acc);
    gateup_epilogue<RGA>(a, d, nb, cnt, acc, C, rsum);
}

template <int RGA>
__device__ __forceinline__ void down_mix_body(const MoeArgs& a, const ItemDesc* d, int nb, int cnt, u32x4_t* stage,
                                              uint32_t* wlds, float* C, float* rsum, int* s_comb) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p0 = d->p0;
    const int tn = a.H / 16;
    MfmaPipeMix<1, RGA> L;
    L.tn = tn;
    L.nsteps = a.I / 32;
    L.lds = stage;
    L.lane = lane;
    L.wl = wlds + wave * 8 * kMixTS;
    L.wrs = buffer_rsrc(reinterpret_cast<const void*>(d->tab[6]));
    L.krs = buffer_rsrc(reinterpret_cast<const void*>(d->km[4]));
    L.ors = buffer_rsrc(reinterpret_cast<const void*>(d->km[5]));
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
        int ct = nb * 16 + 4 * wave + 2 * pr;
        L.col[pr] = ct < tn ? ct : tn - 2;             // a last half block: in-bounds loads, results unused
    }
    L.setup_a(cnt, [&](int, int row) { return reinterpret_cast<const _Float16*>(a.abuf) + (size_t)(p0 + row) * a.I; });
    f4_t acc[kMfT][RGA];
#pragma unroll
    for (int t = 0; t < kMfT; ++t)
#pragma unroll
        for (int rg = 0; rg < RGA; ++rg) acc[t][rg] = f4_t{0.f, 0.f, 0.f, 0.f};
    L.run(acc);
    down_epilogue<RGA>(a, d, nb, cnt, acc, C, rsum, s_comb);
}

template <int RGA>
__global__ __launch_bounds__(256, EXL3_MIX_OCC(RGA)) void gateup_mix_kernel(MoeArgs a) {
    constexpr int CL = RGA == 1 ? 0 : RGA == 2 ? 1 : 2;
    // the epilogue's C reuses the pipeline's A stages and weight slots (dead once the pipeline has drained)
    constexpr int kStage = 4 * (RGA == 1 ? 4 : 2 * RGA) * 64 * 16, kW = 4 * 8 * kMixTS * 4, kC = 2 * 16 * 128 * 4;
    __shared__ __attribute__((aligned(16))) char smem[kStage + kW > kC ? kStage + kW : kC];
    u32x4_t* stage = reinterpret_cast<u32x4_t*>(smem);
    uint32_t* wlds = reinterpret_cast<uint32_t*>(smem + kStage);
    float* C = reinterpret_cast<float*>(smem);
    __shared__ float rsum[2 * 64];
    const int nbI = a.I / 128;
    int idx, nb;
    xcd_map(nbI, idx, nb);
    if (idx >= a.cls_cnt[CL]) return;
    const ItemDesc* d = a.blocks + a.cls_list[CL * a.max_blocks + idx];
    const int cnt = d->cnt;
    const int nblk = a.H / 128;
    for (int i = threadIdx.x; i < 2 * 64; i += 256) {
        const int p = i >> 6, m = i & 63;
        rsum[i] = m < cnt ? sum_ordered(a.xsum + ((size_t)(d->p0 + m) * 2 + p) * nblk, nblk) : 0.f;
    }
    __syncthreads();
    gateup_mix_body<RGA>(a, d, nb, cnt, stage, wlds, C, rsum);
}

template <int RGA>
__global__ __launch_bounds__(256, EXL3_MIX_OCC(RGA)) void down_mix_kernel(MoeArgs a) {
    constexpr int CL = RGA == 1 ? 0 : RGA == 2 ? 1 : 2;
    constexpr int kStage = 4 * (RGA == 1 ? 4 : RGA) * 64 * 16, kW = 4 * 8 * kMixTS * 4, kC = 16 * 256 * 4;
    __shared__ __attribute__((aligned(16))) char smem[kStage + kW > kC ? kStage + kW : kC];   // C aliases, as above
    u32x4_t* stage = reinterpret_cast<u32x4_t*>(smem);
    uint32_t* wlds = reinterpret_cast<uint32_t*>(smem + kStage);
    float* C = reinterpret_cast<float*>(smem);
    __shared__ float rsum[64];
    __shared__ int s_comb[2 * 64];
    const int nbH2 = (a.H / 128 + 1) / 2;
    int idx, nb;
    xcd_map(nbH2, idx, nb);
    if (idx >= a.cls_cnt[CL]) return;
    const ItemDesc* d = a.blocks + a.cls_list[CL * a.max_blocks + idx];
    const int cnt = d->cnt;
    const int nbI = a.I / 128;
    for (int m = threadIdx.x; m < 64; m += 256)
        rsum[m] = m < cnt ? sum_ordered(a.asum + (size_t)(d->p0 + m) * nbI, nbI) : 0.f;
    __syncthreads();
    down_mix_body<RGA>(a, d, nb, cnt, stage, wlds, C, rsum, s_comb);
}

// ------------------------------------------------------------------------------------------------ dense linear
// exl3_gemm for more rows than the GEMV takes per pass: y = Hn(Hk(x * suh) @ W_hat) * svh with the trellis decoded
// straight into MFMA B fragments once per row block (up to 64 rows), as in the reference's large-M linear
// (glm/xpu/csrc/exl3_ops.sycl:643-757), which reconstructs 16384-column fp16 slices and runs a GEMM instead.
//   linear_had   xh[s][m][k] = fp16(H128(fp16(x * suh[s])) / sqrt(128)) and the 128-blocks' sums xsum[s][m][k / 128]
//                (the Hadamard on MFMA, as in the MoE input transform; 16 rows per wave)
//                for every shard s (a fused multi-projection linear: output column blocks of S projections that share
//                the input, each with its own input signs suh[s]; shard_of_nb maps 128-column blocks to shards)
//   linear_mfma  workgroup per (row block, k-split, 256-column block); a wave owns four tile columns. With one split
//                the epilogue writes y; otherwise it writes fp32 partials (affine applied)
//   linear_reduce (k-split only) wave per (row, 128 columns): partials in split order, Hadamard, * svh -> y
struct LinArgs {
    const _Float16* xh;                              // [S][m][k]
    const float* xsum;                               // [S][m][k / 128]
    const int32_t* sonb;                             // shard of each 128-column block (S > 1), else null
    int S;
    const uint32_t* tr;
    const uint16_t* svh;
    void* out;
    int64_t out_ld;
    float* part;                                     // [P][m][n] when P > 1
    int m, k, n, nblk;
    int nrb, ncb, P, bps;                            // row blocks, 256-column blocks, k-splits, 128-blocks per split
    int f32;
};

__global__ __launch_bounds__(256) void linear_had_kernel(const uint16_t* __restrict__ x, int64_t x_ld, int m, int k,
                                                         const uint16_t* __restrict__ suh, _Float16* xh, float* xsum) {
    __shared__ __attribute__((aligned(16))) _Float16 s_out[4][16][136];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kb = blockIdx.y, nblk = k / 128;
    suh += (size_t)blockIdx.z * k;                               // shard s = blockIdx.z
    xh += (size_t)blockIdx.z * m * k;
    xsum += (size_t)blockIdx.z * m * nblk;
    const int r0 = blockIdx.x * 64 + 16 * wave;                  // this wave's 16 rows
    if (r0 >= m) return;
    const int mm = lane & 15, g = lane >> 4;
    const int row = r0 + mm < m ? r0 + mm : m - 1;               // rows past m repeat the last one (not stored)
    const uint16_t* xr = x + (int64_t)row * x_ld + kb * 128 + 8 * g;
    const bool vx = ((uintptr_t)x & 15) == 0 && (x_ld & 7) == 0;
    h8_t xv[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) xv[ks] = load_h8(xr + 32 * ks, vx);
    const h8_t F[2] = {had_fragment(lane, 0), had_fragment(lane, 1)};
    const uint16_t* sv = suh + kb * 128 + 8 * g;
    float part[4];
    had16_rows(xv, sv, ((uintptr_t)sv & 15) == 0, F, lane, s_out[wave], part);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int u = lane + 64 * c, rr = u >> 4, ch = u & 15;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&s_out[wave][rr][8 * ch]);
        if (r0 + rr < m) *reinterpret_cast<u32x4_t*>(xh + (size_t)(r0 + rr) * k + kb * 128 + 8 * ch) = v;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float v = row16_sum(part[i]);
        if (mm == 0 && r0 + 4 * g + i < m) xsum[(size_t)(r0 + 4 * g + i) * nblk + kb] = v;
    }
}

__device__ __forceinline__ void linear_store(const LinArgs& a, int row, int col, float v0, float v1) {
    if (a.f32) {
        float* o = reinterpret_cast<float*>(a.out) + (int64_t)row * a.out_ld + col;
        o[0] = v0;
        o[64] = v1;
    } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + (int64_t)row * a.out_ld + col;
        o[0] = f2h(v0);
        o[64] = f2h(v1);
    }
}

// NPS = 2 for several shards: the two 128-column halves of the block may read different shards' inputs, so both
// are staged and waves 0, 1 (first half) read plane 0, waves 2, 3 plane 1.
template <int K, int RGA, int NPS>
__global__ __launch_bounds__(256, RGA == 1 ? 4 : RGA == 2 ? 3 : 2) void linear_mfma_kernel(LinArgs a) {
    __shared__ u32x4_t stage[4 * (RGA == 1 ? 4 : NPS * RGA) * 64];   // [4 stages][planes][16 RGA rows x 4 units]
                                                                    // (per wave at one row group)
    __shared__ uint32_t wlds[4 * 8 * (8 * K + 4)];       // per wave: 8 staged tiles
    __shared__ float C[16 * 256];
    __shared__ float rsum[NPS][16 * RGA];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int blk, nb;
    xcd_map(a.ncb, blk, nb);
    if (blk >= a.nrb * a.P) return;
    const int rb = blk / a.P, p = blk - rb * a.P;
    const int r0 = rb * 16 * RGA;
    const int cnt = a.m - r0 < 16 * RGA ? a.m - r0 : 16 * RGA;
    const int kb0 = p * a.bps, nkb = a.nblk - kb0 < a.bps ? a.nblk - kb0 : a.bps;
    const int tn = a.n / 16;
    const int nhalf = 2 * nb + 1 < a.n / 128 ? 2 : 1;
    // output scales of the two 128-column halves (unconditional loads, unused past nhalf)
    const uint16_t* sv = a.svh + nb * 256;
    float sd[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int hh = h < nhalf ? h : 0;
        sd[h][0] = h2f(ldg(sv + 128 * hh + lane)) * kRsqrt128;
        sd[h][1] = h2f(ldg(sv + 128 * hh + lane + 64)) * kRsqrt128;
    }
    // shard of each staged plane (plane p: the block's 128-column half p; clamped into [0, S))
    int shard[NPS];
#pragma unroll
    for (int q = 0; q < NPS; ++q) {
        int v = 0;
        if (NPS > 1) {
            v = a.sonb[2 * nb + (q < nhalf ? q : 0)];
            v = v < 0 ? 0 : (v >= a.S ? a.S - 1 : v);
        }
        shard[q] = v;
    }
    if (threadIdx.x < NPS * 16 * RGA) {                // the rows' sums over this split's 128-blocks, per plane
        const int q = threadIdx.x / (16 * RGA), r = threadIdx.x - q * 16 * RGA;
        rsum[q][r] = sum_ordered(a.xsum + ((size_t)shard[q] * a.m + r0 + (r < cnt ? r : cnt - 1)) * a.nblk + kb0, nkb);
    }
    __syncthreads();
    MfmaPipe<K, 1, RGA, NPS> L;
    L.nsteps = nkb * 4;
    L.lds = stage;
    L.lane = lane;
    L.apl = NPS > 1 ? (wave >> 1) : 0;
    const uint32_t* trk = a.tr + (size_t)kb0 * 8 * tn * (8 * K);
    L.setup_w(tn, wlds + wave * 8 * (8 * K + 4), trk, [&](int pair) {
        const int ct = nb * 16 + 4 * wave + 2 * pair;
        return ct < tn ? ct : tn - 2;                  // a last half block: in-bounds loads, results unused
    });
    L.setup_a(cnt, [&](int q, int row) {                 // a select, not an index: shard[] stays in registers
        const int sq = (NPS > 1 && q != 0) ? shard[NPS - 1] : shard[0];
        return a.xh + ((size_t)sq * a.m + r0 + row) * a.k + kb0 * 128;
    });
    f4_t acc[kMfT][RGA];
#pragma unroll
    for (int t = 0; t < kMfT; ++t)
#pragma unroll
        for (int rg = 0; rg < RGA; ++rg) acc[t][rg] = f4_t{0.f, 0.f, 0.f, 0.f};
    L.run(acc);
    const bool single = a.P == 1;
    float* part = a.part + (size_t)p * a.m * a.n;
#pragma unroll
    for (int rg = 0; rg < RGA; ++rg) {
#pragma unroll
        for (int t = 0; t < kMfT; ++t) {
            const int col = (4 * wave + t) * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) C[(4 * (lane >> 4) + i) * 256 + col] = acc[t][rg][i];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 8; ++j) {                 // (row, half) pairs of this wave
            const int ml = 4 * wave + (j >> 1), h = j & 1, m = 16 * rg + ml;
            if (m >= cnt || h >= nhalf) continue;
            const float sx = kMul1C2 * rsum[NPS > 1 ? h : 0][m];
            float v0 = kMul1C1 * C[ml * 256 + 128 * h + lane] + sx, v1 = kMul1C1 * C[ml * 256 + 128 * h + lane + 64] + sx;
            const int col = nb * 256 + 128 * h + lane;
            if (single) {
                fwht128_wave(v0, v1, lane);
                linear_store(a, r0 + m, col, v0 * sd[h][0], v1 * sd[h][1]);
            } else {
                float* dst = part + (size_t)(r0 + m) * a.n + col;
                dst[0] = v0;
                dst[64] = v1;
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------ host
typedef void (*mfma_fn)(MoeArgs);

// Raise a kernel's dynamic-LDS limit once (the attribute is per function).
static hipError_t set_max_lds(const void* fn, int bytes) {
    static const void* done[64];
    static int ndone = 0;
    for (int i = 0; i < ndone; ++i)
        if (done[i] == fn) return hipSuccess;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && ndone < 64) done[ndone++] = fn;
    return e;
}

// PLANAR4 instantiations where that order differs from tile order (K = 3, 5, 6, 7)
template <int RGA>
static mfma_fn pick_gu(int K, bool pl) {
    if (pl) {
        switch (K) {
            case 3: return gateup_mfma_kernel<3, RGA, true>;
            case 5: return gateup_mfma_kernel<5, RGA, true>;
            case 6: return gateup_mfma_kernel<6, RGA, true>;
            case 7: return gateup_mfma_kernel<7, RGA, true>;
            default: break;
        }
    }
    switch (K) {
        case 1: return gateup_mfma_kernel<1, RGA>;
        case 2: return gateup_mfma_kernel<2, RGA>;
        case 3: return gateup_mfma_kernel<3, RGA>;
        case 4: return gateup_mfma_kernel<4, RGA>;
        case 5: return gateup_mfma_kernel<5, RGA>;
        case 6: return gateup_mfma_kernel<6, RGA>;
        case 7: return gateup_mfma_kernel<7, RGA>;
        default: return gateup_mfma_kernel<8, RGA>;
    }
}

template <int RGA>
static mfma_fn pick_dn(int K, bool pl) {
    if (pl) {
        switch (K) {
            case 3: return down_mfma_kernel<3, RGA, true>;
            case 5: return down_mfma_kernel<5, RGA, true>;
            case 6: return down_mfma_kernel<6, RGA, true>;
            case 7: return down_mfma_kernel<7, RGA, true>;
            default: break;
        }
    }
    switch (K) {
        case 1: return down_mfma_kernel<1, RGA>;
        case 2: return down_mfma_kernel<2, RGA>;
        case 3: return down_mfma_kernel<3, RGA>;
        case 4: return down_mfma_kernel<4, RGA>;
        case 5: return down_mfma_kernel<5, RGA>;
        case 6: return down_mfma_kernel<6, RGA>;
        case 7: return down_mfma_kernel<7, RGA>;
        default: return down_mfma_kernel<8, RGA>;
    }
}

template <typename F>
static int fork3(hipStream_t st, F launch) {
    // the three row classes run concurrently: 4 row groups on the caller's stream, 2 and 1 on the side streams
    if (env_int("EXL3MI_SERIAL_CLASSES", 0)) {            // every class on the caller's stream, one after another
        int rc = 0;
        if ((rc = launch(4, st)) || (rc = launch(2, st)) || (rc = launch(1, st))) return rc;
        return EXL3_OK;
    }
    AuxStreams ax;
    int rc = aux_streams(&ax);
    if (rc) return rc;
    EXL3_CHECK_HIP(hipEventRecord(ax.ev[0], st));
    EXL3_CHECK_HIP(hipStreamWaitEvent(ax.s[0], ax.ev[0], 0));
    EXL3_CHECK_HIP(hipStreamWaitEvent(ax.s[1], ax.ev[0], 0));
    if ((rc = launch(4, st)) || (rc = launch(2, ax.s[0])) || (rc = launch(1, ax.s[1]))) return rc;
    EXL3_CHECK_HIP(hipEventRecord(ax.ev[1], ax.s[0]));
    EXL3_CHECK_HIP(hipEventRecord(ax.ev[2], ax.s[1]));
    EXL3_CHECK_HIP(hipStreamWaitEvent(st, ax.ev[1], 0));
    EXL3_CHECK_HIP(hipStreamWaitEvent(st, ax.ev[2], 0));
    return EXL3_OK;
}

// The grouped GEMM of one layer call: the input transform, then per row class gate|up followed by down on that class's
// stream (a class's down blocks read only the down inputs its own gate|up blocks wrote; tokens whose slots span
// classes are combined by the last slot to finish), so one class's down pass overlaps the others' gate|up.
int launch_moe_mfma(const MoeArgs& a, hipStream_t st) {
    const int nxb = (a.max_blocks + 7) / 8 * 8;
    const int64_t had_jobs = (int64_t)(a.M * a.slots + 15) / 16 * (a.H / 128);
    EXL3_CHECK_ARG(had_jobs / 4 < 0x7FFFFFFF, "exl3_moe_forward: too many rows");
    EXL3_LAUNCH("moe_pairs_had", pairs_had_kernel, dim3((unsigned)((had_jobs + 3) / 4)), dim3(256), 0, st, a);
    const dim3 grid_gu(nxb * (a.I / 128)), grid_dn(nxb * ((a.H / 128 + 1) / 2));
    return fork3(st, [&](int rga, hipStream_t s) -> int {
        mfma_fn gu = a.Kg == 0 ? (rga == 4 ? gateup_mix_kernel<4> : rga == 2 ? gateup_mix_kernel<2> : gateup_mix_kernel<1>)
                               : (rga == 4 ? pick_gu<4>(a.Kg, a.planar) : rga == 2 ? pick_gu<2>(a.Kg, a.planar)
                                            : pick_gu<1>(a.Kg, a.planar));
        mfma_fn dn = a.Kd == 0 ? (rga == 4 ? down_mix_kernel<4> : rga == 2 ? down_mix_kernel<2> : down_mix_kernel<1>)
                               : (rga == 4 ? pick_dn<4>(a.Kd, a.planar) : rga == 2 ? pick_dn<2>(a.Kd, a.planar)
                                            : pick_dn<1>(a.Kd, a.planar));
        EXL3_LAUNCH(rga == 4 ? "moe_gateup_mfma_r4" : rga == 2 ? "moe_gateup_mfma_r2" : "moe_gateup_mfma_r1", gu,
                    grid_gu, dim3(256), 0, s, a);
        EXL3_LAUNCH(rga == 4 ? "moe_down_mfma_r4" : rga == 2 ? "moe_down_mfma_r2" : "moe_down_mfma_r1", dn, grid_dn,
                    dim3(256), 0, s, a);
        return EXL3_OK;
    });
}

// Split-K finish: wave per (row, 128-column block): the split partials summed in split order (eight splits' loads in
// flight at a time), Hadamard, * svh / sqrt(128).
__global__ __launch_bounds__(256) void linear_reduce_kernel(LinArgs a) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row = blockIdx.x * 4 + wave;
    if (row >= a.m) return;
    const int col = blockIdx.y * 128 + lane;
    const float s0 = h2f(ldg(a.svh + col)) * kRsqrt128, s1 = h2f(ldg(a.svh + col + 64)) * kRsqrt128;
    const float* q = a.part + (size_t)row * a.n + col;
    const size_t ps = (size_t)a.m * a.n;
    float v0 = 0.f, v1 = 0.f;
    for (int p0 = 0; p0 < a.P; p0 += 8) {
        float t0[8], t1[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int pp = p0 + i < a.P ? p0 + i : a.P - 1;
            t0[i] = ldg(q + pp * ps);
            t1[i] = ldg(q + pp * ps + 64);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (p0 + i < a.P) {
                v0 += t0[i];
                v1 += t1[i];
            }
    }
    fwht128_wave(v0, v1, lane);
    linear_store(a, row, col, v0 * s0, v1 * s1);
}

typedef void (*lin_fn)(LinArgs);

template <int RGA, int NPS>
static lin_fn pick_lin(int K) {
    switch (K) {
        case 1: return linear_mfma_kernel<1, RGA, NPS>;
        case 2: return linear_mfma_kernel<2, RGA, NPS>;
        case 3: return linear_mfma_kernel<3, RGA, NPS>;
        case 4: return linear_mfma_kernel<4, RGA, NPS>;
        case 5: return linear_mfma_kernel<5, RGA, NPS>;
        case 6: return linear_mfma_kernel<6, RGA, NPS>;
        case 7: return linear_mfma_kernel<7, RGA, NPS>;
        default: return linear_mfma_kernel<8, RGA, NPS>;
    }
}

template <int NPS>
static lin_fn pick_lin_rga(int RGA, int K) {
    return RGA == 4 ? pick_lin<4, NPS>(K) : RGA == 2 ? pick_lin<2, NPS>(K) : pick_lin<1, NPS>(K);
}

// Dense linear on MFMA (m > the GEMV's rows per pass). Row blocks of 16, 32 or 64 rows (by m); k-splits so that the
// grid covers about the workgroups the device holds at once, each split at least two 128-blocks of k.
int launch_linear_mfma(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const uint32_t* tr, int64_t n, int K,
                       void* C, int64_t c_ld, bool f32, const uint16_t* suh, int S, const int32_t* sonb,
                       const uint16_t* svh, hipStream_t st) {
    const int RGA = m <= 16 ? 1 : m <= 32 ? 2 : 4;
    const int R = 16 * RGA;
    const int nblk = (int)(k / 128);
    if (m > 0x7FFFFFFF / 64 || k > 0x7FFFFFFF || n > 0x7FFFFFFF || nblk > 65535)
        return fail(EXL3_ERR_INVALID, "exl3_gemm: shape too large");
    LinArgs a;
    a.m = (int)m;
    a.k = (int)k;
    a.n = (int)n;
    a.nblk = nblk;
    a.nrb = (int)((m + R - 1) / R);
    a.ncb = (int)((n + 255) / 256);
    lin_fn fn = S > 1 ? pick_lin_rga<2>(RGA, K) : pick_lin_rga<1>(RGA, K);
    int resident = 0;
    int rc = resident_blocks((const void*)fn, 256, &resident);
    if (rc) return rc;
    const int target = env_int("EXL3MI_LINEAR_JOBS", resident);
    const int64_t tiles = (int64_t)a.nrb * a.ncb;
    int P = (int)((target + tiles - 1) / tiles);
    const int pmax = nblk / 2 > 1 ? nblk / 2 : 1;
    P = P < 1 ? 1 : (P > pmax ? pmax : P);
    a.bps = (nblk + P - 1) / P;
    a.P = (nblk + a.bps - 1) / a.bps;
    const size_t xh_b = carve_size((size_t)S * m * k, 2), xs_b = carve_size((size_t)S * m * nblk, 4);
    const size_t part_b = a.P > 1 ? carve_size((size_t)a.P * m * n, 4) : 0;
    Workspace ws;
    rc = workspace(xh_b + xs_b + part_b, 0, st, &ws);
    if (rc) return rc;
    Carve cv{ws.scratch, ws.scratch_bytes};
    _Float16* xh = cv.take<_Float16>((size_t)S * m * k);
    float* xsum = cv.take<float>((size_t)S * m * nblk);
    a.part = a.P > 1 ? cv.take<float>((size_t)a.P * m * n) : nullptr;
    if (!xh || !xsum || (a.P > 1 && !a.part)) return fail(EXL3_ERR_INVALID, "exl3_gemm: workspace carve failed");
    a.xh = xh;
    a.xsum = xsum;
    a.S = S;
    a.sonb = S > 1 ? sonb : nullptr;
    a.tr = tr;
    a.svh = svh;
    a.out = C;
    a.out_ld = c_ld;
    a.f32 = f32 ? 1 : 0;
    const dim3 hgrid((unsigned)((m + 63) / 64), (unsigned)nblk, (unsigned)S);
    EXL3_LAUNCH("linear_had", linear_had_kernel, hgrid, dim3(256), 0, st, A, a_ld, (int)m, (int)k, suh, xh, xsum);
    const int64_t nx = ((int64_t)a.nrb * a.P + 7) / 8 * 8 * a.ncb;
    if (nx > 0x7FFFFFFF) return fail(EXL3_ERR_INVALID, "exl3_gemm: grid too large");
    EXL3_LAUNCH("linear_mfma", fn, dim3((unsigned)nx), dim3(256), 0, st, a);
    if (a.P > 1)
        EXL3_LAUNCH("linear_reduce", linear_reduce_kernel, dim3((unsigned)((m + 3) / 4), (unsigned)(n / 128)),
                    dim3(256), 0, st, a);
    return EXL3_OK;
}

}  // namespace exl3
