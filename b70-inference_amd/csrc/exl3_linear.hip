// EXL3 dense linear on gfx950: reconstruct, blockwise Hadamard, and the small-M decode GEMV.
//
// Reference semantics: exllamav3 reconstruct_slice / had_r_128 / exl3_gemm (ext-op-inventory.md:498-612) and the
// XPU library's exl3_reconstruct / exl3_gemm_small (glm/xpu/csrc/exl3_ops.sycl:258-321, 539-555).
#include "exl3_device.h"
#include "exl3_gemv.h"

#include <mutex>
#include "exl3_runtime.h"

namespace exl3 {

// ================================================================================================ reconstruct
// One wave per (128-column strip, tile-row): lanes decode their chunks, stage the 16 x 128 fp16 block in LDS, then
// write it out with 16-byte row stores.
template <int K>
__global__ __launch_bounds__(64) void reconstruct_kernel(const uint32_t* __restrict__ tr, int tn, int n0_tiles,
                                                         uint16_t* __restrict__ out, int64_t out_ld) {
    __shared__ __attribute__((aligned(16))) uint16_t blk[16][136];
    const int lane = threadIdx.x;
    const int strip = blockIdx.x, trow = blockIdx.y;
    const uint32_t* p = tr + ((size_t)trow * tn + n0_tiles + (size_t)strip * 8) * (8 * K);
    uint32_t R[K + 1];
    load_chunk<K>(p, lane, R);
    chunk_prev<K>(lane, R);
    h2_t w[16];
    decode_chunk<K>(R, w);
    const int cbase = 16 * (lane >> 3) + (lane & 7);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int r = pos_row(2 * j), c = cbase + 8 * pos_half(2 * j);
        const uint32_t v = __builtin_bit_cast(uint32_t, w[j]);   // element 0 in the low half
        blk[r][c] = (uint16_t)(v & 0xFFFFu);
        blk[r + 1][c] = (uint16_t)(v >> 16);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = i * 64 + lane, r = idx >> 4, c8 = idx & 15;
        uint4 v = *reinterpret_cast<const uint4*>(&blk[r][c8 * 8]);
        *reinterpret_cast<uint4*>(out + (size_t)(16 * trow + r) * out_ld + (size_t)strip * 128 + c8 * 8) = v;
    }
}

// ================================================================================================ reconstruct_had
// Original-basis weight slice W = diag(suh) Hblk W_hat Hblk diag(svh) (Hblk = blockdiag(H128 / sqrt(128))): one
// workgroup per 128 x 128 block. The block's 8 tile-row strips are decoded into LDS (fp32), every column gets the
// 128-point transform (one wave per column), then every row (one wave per row), which also applies
// suh[row] * svh[col] / 128 and rounds once to fp16. All of it in fp32: within one fp16 rounding of the exact weight.
template <int K>
__global__ __launch_bounds__(256) void reconstruct_had_kernel(const uint32_t* __restrict__ tr, int tn, int n0_tiles,
                                                              const uint16_t* __restrict__ suh,
                                                              const uint16_t* __restrict__ svh,
                                                              uint16_t* __restrict__ out, int64_t out_ld) {
    __shared__ float M[128][129];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = blockIdx.x, kb = blockIdx.y;
    const int cbase = 16 * (lane >> 3) + (lane & 7);
    for (int s = wave; s < 8; s += 4) {                         // tile-row strips of the block
        const uint32_t* p = tr + ((size_t)(8 * kb + s) * tn + n0_tiles + (size_t)nb * 8) * (8 * K);
        uint32_t R[K + 1];
        load_chunk<K>(p, lane, R);
        chunk_prev<K>(lane, R);
        h2_t w[16];
        decode_chunk<K>(R, w);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int r = 16 * s + pos_row(2 * j), c = cbase + 8 * pos_half(2 * j);
            M[r][c] = (float)w[j][0];
            M[r + 1][c] = (float)w[j][1];
        }
    }
    __syncthreads();
    for (int c = wave; c < 128; c += 4) {                       // Hblk W_hat: transform every column
        float a = M[lane][c], b = M[lane + 64][c];
        fwht128_wave(a, b, lane);
        M[lane][c] = a;
        M[lane + 64][c] = b;
    }
    __syncthreads();
    const float s0 = h2f(ldg(svh + nb * 128 + lane)), s1 = h2f(ldg(svh + nb * 128 + lane + 64));
    for (int r = wave; r < 128; r += 4) {                       // (..) Hblk: transform every row, then the signs
        float a = M[r][lane], b = M[r][lane + 64];
        fwht128_wave(a, b, lane);
        const float su = h2f(ldg(suh + kb * 128 + r)) * (1.0f / 128.0f);
        uint16_t* o = out + (size_t)(kb * 128 + r) * out_ld + nb * 128;
        o[lane] = f2h(a * su * s0);
        o[lane + 64] = f2h(b * su * s1);
    }
}

// ================================================================================================ had_r_128
template <bool F16>
__global__ __launch_bounds__(64) void had_kernel(const void* __restrict__ in, int64_t in_ld, void* __restrict__ out,
                                                 int64_t out_ld, const uint16_t* __restrict__ pre,
                                                 const uint16_t* __restrict__ post, float r) {
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int c0 = blockIdx.y * 128 + lane, c1 = c0 + 64;
    float a, b;
    if (F16) {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(in) + row * in_ld;
        a = h2f(src[c0]);
        b = h2f(src[c1]);
        if (pre) {
            a = (float)(_Float16)(a * h2f(pre[c0]));
            b = (float)(_Float16)(b * h2f(pre[c1]));
        }
    } else {
        const float* src = reinterpret_cast<const float*>(in) + row * in_ld;
        a = src[c0];
        b = src[c1];
        if (pre) {
            a *= h2f(pre[c0]);
            b *= h2f(pre[c1]);
        }
    }
    fwht128_wave(a, b, lane);
    a *= r;
    b *= r;
    if (F16) {
        a = (float)(_Float16)a;
        b = (float)(_Float16)b;
        if (!pre && post) {
            a = (float)(_Float16)(a * h2f(post[c0]));
            b = (float)(_Float16)(b * h2f(post[c1]));
        }
        uint16_t* dst = reinterpret_cast<uint16_t*>(out) + row * out_ld;
        dst[c0] = f2h(a);
        dst[c1] = f2h(b);
    } else {
        if (!pre && post) {
            a *= h2f(post[c0]);
            b *= h2f(post[c1]);
        }
        float* dst = reinterpret_cast<float*>(out) + row * out_ld;
        dst[c0] = a;
        dst[c1] = b;
    }
}

// ================================================================================================ dense GEMV
// Workgroup = 4 waves on one 128-column strip and one k-split (a run of Hadamard blocks). Phase 1 computes the
// split's transformed activations into LDS; phase 2 streams the strip's tile-rows (wave w takes tile-rows w, w+4,..);
// phase 3 reduces the waves in LDS and, across splits, either through per-strip partials and an arrival counter (the
// last workgroup of a strip sums the partials in split order, deterministic) or through tagged partials (`tag`): each
// partial is stored as the word bits(v) ^ kPartEmpty, so that a zero word means "not written yet" (kPartEmpty is a
// signalling NaN, which no arithmetic result is), and the strip's last split polls for the others' words, sums them
// in split order, clears them to zero and finishes the strip. The tagged form has no arrival round trip (no store
// drain, no atomic) on the path; its wait is bounded (spin_max polls, then the status word is set). Either way the
// last step applies the output Hadamard and svh.
constexpr uint32_t kPartEmpty = 0x7FBFDEADu;

struct GemvArgs {
    const uint16_t* x;
    int64_t x_ld;
    int m;
    const uint32_t* tr;
    int tn;
    const uint16_t* suh;                             // [S][k]
    const int32_t* sonb;                             // shard of each 128-column strip (S > 1), else null
    int S;
    const uint16_t* svh;
    void* out;
    int64_t out_ld;
    float* part;
    int* cnt;
    int P;
    int nblk;
    // multi-matrix mode (exl3_mgemm; trp == null otherwise): slot z = blockIdx.z runs matrix q = idx[z] (z without
    // idx; with qmin >= 0 only q in [qmin, qmax), rebased by qmin; slots whose q falls outside [0, nmat) are skipped)
    // on A batch z / a_div (x_bs = 0 broadcasts) into out + z * out_bs, with its own partials and counters
    const int64_t* trp;
    const int64_t* suhp;
    const int64_t* svhp;
    const int64_t* idx;
    int nmat;
    int a_div;
    int64_t qmin, qmax;
    int64_t x_bs, out_bs;
    // tagged partials [strips][P][128] (zero between calls), one row and one slot (gridDim.z == 1); null: arrival
    // counters
    uint32_t* tag;
    int* status;                                     // set when the tagged wait gives up
    int spin_max;
};

// Matrix of multi-matrix slot z (-1: skipped).
__device__ __forceinline__ int64_t mgemm_matrix(const int64_t* idx, int z, int64_t qmin, int64_t qmax, int nmat) {
    int64_t q = idx ? idx[z] : z;
    if (qmin >= 0) q = (q >= qmin && q < qmax) ? q - qmin : -1;
    return (q >= 0 && q < nmat) ? q : -1;
}

template <int K, int M, bool F32, int NW>
__global__ __launch_bounds__(64 * NW) void gemv_kernel(GemvArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[M][kGemvKBMax * 128];
    __shared__ float red[NW][M][2][64];
    __shared__ float bsum[M][kGemvKBMax];
    __shared__ int s_last;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int strip = blockIdx.x, p = blockIdx.y, z = blockIdx.z;
    const uint32_t* tr = a.tr;
    const uint16_t* suh_all = a.suh;
    const uint16_t* svh = a.svh;
    if (a.trp) {
        const int64_t q = mgemm_matrix(a.idx, z, a.qmin, a.qmax, a.nmat);
        if (q < 0) return;                                          // uniform: the whole workgroup leaves
        tr = reinterpret_cast<const uint32_t*>(a.trp[q]);
        suh_all = reinterpret_cast<const uint16_t*>(a.suhp[q]);
        svh = reinterpret_cast<const uint16_t*>(a.svhp[q]);
    }
    const uint16_t* x = a.x + (int64_t)(z / a.a_div) * a.x_bs;
    float* part = a.part + (size_t)z * gridDim.x * a.P * M * 128;
    int* cnt = a.cnt + (size_t)z * gridDim.x;
    const int b0 = (int)((int64_t)p * a.nblk / a.P), b1 = (int)((int64_t)(p + 1) * a.nblk / a.P);
    const int kb = b1 - b0;
    const size_t rs = (size_t)a.tn * (8 * K);                       // words per tile-row
    const uint32_t* sp = tr + (size_t)strip * (64 * K) + (size_t)b0 * 8 * rs;
    // phase 1: xh = fp16(H128(fp16(x * suh)) / sqrt(128)) for rows < m (zero otherwise), and its block sums; the
    // strip's shard selects the sign vector (clamped into [0, S)). The wave's first x blocks and their signs are
    // loaded before the weight prefetch (loads complete in issue order: their transforms then wait for nothing issued
    // after them), with clamped addresses so that no load sits under a branch.
    int shard = 0;
    if (a.sonb) {
        shard = a.sonb[strip];
        shard = shard < 0 ? 0 : (shard >= a.S ? a.S - 1 : shard);
    }
    const uint16_t* suh = suh_all + (size_t)shard * (a.nblk * 128);
    const int nbm = M * kb;                                         // (row, block) pairs of the split
    auto block_ptrs = [&](int i, const uint16_t*& xp, const uint16_t*& sp_) {
        const int m = i / kb, b = i - m * kb, k0 = (b0 + b) * 128;
        xp = x + (int64_t)(m < a.m ? m : 0) * a.x_ld + k0;
        sp_ = suh + k0;
    };
    // Only the wave's first blocks go ahead of the weight prefetch (two up to 4 rows, four above); the rest are
    // loaded after it. Hoisting every block put up to 16 x loads per wave in front of the first weight rows: 4096 x
    // 4096 at 8 rows 14.47 us against 12.84 with four hoisted (3 rows 9.71 against 9.33 with two, one row 6.89 / 6.75).
    constexpr int JB = (M * kGemvKBMax + NW - 1) / NW;              // blocks per wave, at most
    constexpr int JCAP = M <= 4 ? 2 : 4;
    constexpr int JE = JB < JCAP ? JB : JCAP;
    HadIn hv[JE];
#pragma unroll
    for (int j = 0; j < JE; ++j) {
        const int i = wave + j * NW;
        const uint16_t *xp, *sq;
        block_ptrs(i < nbm ? i : nbm - 1, xp, sq);
        hv[j] = had_in_load(xp, sq, lane);
    }
    StripRing<K, kLinearRing> ring;
    // weight loads in flight during phase 1, issued without a branch (wave < NW <= 8 <= kb * 8 tile-rows)
    strip_prefetch<K, kLinearRing, false>(sp, rs, wave, kb * 8, NW, lane, ring);
#pragma unroll
    for (int j = 0; j < JE; ++j) {
        const int i = wave + j * NW;
        if (i < nbm) {
            const int m = i / kb, b = i - m * kb;
            const float s = had_in_finish(hv[j], m < a.m, &xs[m][b * 128], lane);
            if (lane == 0) bsum[m][b] = s;
        }
    }
    for (int i = wave + JE * NW; i < nbm; i += NW) {
        const uint16_t *xp, *sq;
        block_ptrs(i, xp, sq);
        const int m = i / kb, b = i - m * kb;
        const float s = had_in_finish(had_in_load(xp, sq, lane), m < a.m, &xs[m][b * 128], lane);
        if (lane == 0) bsum[m][b] = s;
    }
    __syncthreads();

    // phase 2: decode-in-GEMV over the split's tile-rows
    float acc[M][2];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m][0] = acc[m][1] = 0.f;
    strip_gemv_run<K, M, kLinearRing>(sp, rs, wave, kb * 8, NW, lane, &xs[0][0], kGemvKBMax * 128, acc, ring);

    // phase 3: reduce waves, then splits
#pragma unroll
    for (int m = 0; m < M; ++m) {
        red[wave][m][0][lane] = acc[m][0];
        red[wave][m][1][lane] = acc[m][1];
    }
    __syncthreads();
    const int cbase = 16 * (lane >> 3) + (lane & 7);
    if constexpr (M == 1) {                                     // the tagged exchange serves one-row calls only
        if (a.tag) {
            __shared__ float own[128];                          // the last split's own partial
            uint32_t* tg = a.tag + (size_t)strip * a.P * 128;
            const bool fin = p == a.P - 1;
            if (wave == 0) {
                float sx = 0.f;
                for (int b = 0; b < kb; ++b) sx += bsum[0][b];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float v = red[0][0][h][lane];
#pragma unroll
                    for (int w = 1; w < NW; ++w) v += red[w][0][h][lane];
                    v = kMul1C1 * v + kMul1C2 * sx;
                    const int c = cbase + 8 * h;
                    if (fin) own[c] = v;
                    else __hip_atomic_store(tg + (size_t)p * 128 + c, __builtin_bit_cast(uint32_t, v) ^ kPartEmpty,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            if (!fin) return;
            // polled once the workgroup's own partial is in LDS (polling while wave 0 still reduced it found the
            // other splits' words missing more often, and a miss costs a round trip)
            __syncthreads();
            if (wave != 0) return;
            float sa = 0.f, sb = 0.f;
            // splits 0 .. P - 2 in order, eight at a time: every word of a group loaded before any is checked
            for (int q0 = 0; q0 < a.P - 1; q0 += 8) {
                uint32_t wa[8], wb[8];
                for (int n = 0;;) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int q = q0 + j < a.P - 1 ? q0 + j : q0;   // past the last split: re-read split q0
                        wa[j] = __hip_atomic_load(tg + (size_t)q * 128 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        wb[j] = __hip_atomic_load(tg + (size_t)q * 128 + lane + 64, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
                    }
                    bool miss = false;
#pragma unroll
                    for (int j = 0; j < 8; ++j) miss = miss || wa[j] == 0u || wb[j] == 0u;
                    if (!__ballot(miss)) break;
                    if (++n > a.spin_max) {
                        if (lane == 0) report_timeout(a.status);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (q0 + j < a.P - 1) {
                        sa += __builtin_bit_cast(float, wa[j] ^ kPartEmpty);
                        sb += __builtin_bit_cast(float, wb[j] ^ kPartEmpty);
                    }
            }
            float va = sa + own[lane], vb = sb + own[lane + 64];
            fwht128_wave(va, vb, lane);
            const int c0 = strip * 128 + lane, c1 = c0 + 64;
            va *= kRsqrt128 * h2f(ldg(svh + c0));
            vb *= kRsqrt128 * h2f(ldg(svh + c1));
            if (F32) {
                float* o = reinterpret_cast<float*>(a.out);
                o[c0] = va;
                o[c1] = vb;
            } else {
                uint16_t* o = reinterpret_cast<uint16_t*>(a.out);
                o[c0] = f2h(va);
                o[c1] = f2h(vb);
            }
            // the words back to zero for the next call
            for (int q = 0; q < a.P - 1; ++q) {
                __hip_atomic_store(tg + (size_t)q * 128 + lane, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(tg + (size_t)q * 128 + lane + 64, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return;
        }
    }
    float* mypart = part + ((size_t)strip * a.P + p) * M * 128;
    if (wave == 0) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float sx = 0.f;
            for (int b = 0; b < kb; ++b) sx += bsum[m][b];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float v = red[0][m][h][lane];
#pragma unroll
                for (int w = 1; w < NW; ++w) v += red[w][m][h][lane];
                splitk_store(mypart + m * 128 + cbase + 8 * h, kMul1C1 * v + kMul1C2 * sx);
            }
        }
    }
    if (!splitk_arrive(&cnt[strip], a.P, &s_last)) return;
    for (int m = wave; m < M && m < a.m; m += NW) {
        float va = 0.f, vb = 0.f;
#pragma unroll 8
        for (int pp = 0; pp < a.P; ++pp) {
            const float* q = part + (((size_t)strip * a.P + pp) * M + m) * 128;
            va += splitk_load(q + lane);
            vb += splitk_load(q + lane + 64);
        }
        fwht128_wave(va, vb, lane);
        const int c0 = strip * 128 + lane, c1 = c0 + 64;
        va *= kRsqrt128 * h2f(ldg(svh + c0));
        vb *= kRsqrt128 * h2f(ldg(svh + c1));
        if (F32) {
            float* o = reinterpret_cast<float*>(a.out) + z * a.out_bs + (int64_t)m * a.out_ld;
            o[c0] = va;
            o[c1] = vb;
        } else {
            uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + z * a.out_bs + (int64_t)m * a.out_ld;
            o[c0] = f2h(va);
            o[c1] = f2h(vb);
        }
    }
    if (threadIdx.x == 0) cnt[strip] = 0;
}

// ------------------------------------------------------------------------------------------------ dispatch
typedef void (*gemv_fn)(GemvArgs);

// Waves per workgroup: 4, or 8 for up to 2 rows when the grid is small enough for one round of workgroups (then two
// waves per SIMD share a split's tile-rows: C1, 4096 x 4096 at one row, 7.66 -> 7.29 us; with more workgroups than
// one round, eight-wave workgroups were slower: 5376 x 21504 at one row, 21.0 -> 21.3 us)
constexpr int kGemvWideMaxWG = 512;

template <int K, int M>
static gemv_fn gemv_pick(bool f32, bool wide) {
    if constexpr (M <= 2) {
        if (wide) return f32 ? (gemv_fn)gemv_kernel<K, M, true, 8> : (gemv_fn)gemv_kernel<K, M, false, 8>;
    }
    return f32 ? (gemv_fn)gemv_kernel<K, M, true, 4> : (gemv_fn)gemv_kernel<K, M, false, 4>;
}

template <int K>
static gemv_fn gemv_pick_m(int M, bool f32, bool wide) {
    switch (M) {
        case 1: return gemv_pick<K, 1>(f32, wide);
        case 2: return gemv_pick<K, 2>(f32, wide);
        case 3: return gemv_pick<K, 3>(f32, wide);
        case 4: return gemv_pick<K, 4>(f32, wide);
        case 5: return gemv_pick<K, 5>(f32, wide);
        case 6: return gemv_pick<K, 6>(f32, wide);
        case 7: return gemv_pick<K, 7>(f32, wide);
        default: return gemv_pick<K, 8>(f32, wide);
    }
}

static gemv_fn gemv_select(int K, int M, bool f32, bool wide) {
    switch (K) {
        case 1: return gemv_pick_m<1>(M, f32, wide);
        case 2: return gemv_pick_m<2>(M, f32, wide);
        case 3: return gemv_pick_m<3>(M, f32, wide);
        case 4: return gemv_pick_m<4>(M, f32, wide);
        case 5: return gemv_pick_m<5>(M, f32, wide);
        case 6: return gemv_pick_m<6>(M, f32, wide);
        case 7: return gemv_pick_m<7>(M, f32, wide);
        default: return gemv_pick_m<8>(M, f32, wide);
    }
}

// Number of k-splits: enough workgroups to cover the chip, but at most kGemvMaxSplits (8 for up to 2 rows, 16 for
// more: every split adds a partial row to the last workgroup's reduction, and more rows give each split more work to
// hide it behind; measured over 1024² .. 21504 x 5376 at 1 and 4 rows) and at most kGemvKBMax blocks per split.
static int gemv_splits(int strips, int nblk, int rows) {
    const int target = env_int("EXL3MI_TARGET_WG", kGemvTargetWG);
    int P = (target + strips - 1) / strips;
    const int smax = env_int("EXL3MI_GEMV_MAX_SPLITS", rows <= 2 ? kGemvMaxSplits : 2 * kGemvMaxSplits);
    if (P > smax) P = smax;
    int pmin = (nblk + kGemvKBMax - 1) / kGemvKBMax;
    if (P < pmin) P = pmin;
    if (P > nblk) P = nblk;
    return P < 1 ? 1 : P;
}

// Dense linear on MFMA (exl3_mfma.hip), used from kLinearMfmaMinRows rows on.
int launch_linear_mfma(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const uint32_t* tr, int64_t n, int K,
                       void* C, int64_t c_ld, bool f32, const uint16_t* suh, int S, const int32_t* sonb,
                       const uint16_t* svh, hipStream_t st);
constexpr int kLinearMfmaMinRows = 9;

// Launches over chunks of up to kGemvMaxRows rows of `ga` (x, out and m describe all rows; the workspace holds
// slots x strips x P partial blocks and slots x strips counters).
// With `profiled` false the launches bypass the opt-in event profiler (which creates events), so that the
// allocation-free entry point never allocates.
static int gemv_chunks(GemvArgs ga, int64_t m, int K, bool f32, int strips, int slots, hipStream_t st,
                       bool profiled = true) {
    const int Mmax = kGemvMaxRows;
    for (int64_t m0 = 0; m0 < m; m0 += Mmax) {
        const int mm = (int)((m - m0) < Mmax ? (m - m0) : Mmax);
        GemvArgs c = ga;
        c.x = ga.x + m0 * ga.x_ld;
        c.m = mm;
        c.out = f32 ? (void*)(reinterpret_cast<float*>(ga.out) + m0 * ga.out_ld)
                    : (void*)(reinterpret_cast<uint16_t*>(ga.out) + m0 * ga.out_ld);
        const bool wide = mm <= 2 && (int64_t)strips * ga.P * slots <= kGemvWideMaxWG;
        gemv_fn fn = gemv_select(K, mm, f32, wide);
        const dim3 block(wide ? 512 : 256);
        if (profiled) {
            EXL3_LAUNCH("gemv", fn, dim3(strips, ga.P, slots), block, 0, st, c);
        } else {
            hipLaunchKernelGGL(fn, dim3(strips, ga.P, slots), block, 0, st, c);
            EXL3_CHECK_HIP(hipGetLastError());
        }
    }
    return EXL3_OK;
}

// Arguments of a dense decode GEMV over all of x's rows, partials and counters left to the caller.
static GemvArgs gemv_args(const uint16_t* A, int64_t a_ld, int64_t k, const uint32_t* tr, int64_t n, void* C,
                          int64_t c_ld, const uint16_t* suh, int S, const int32_t* sonb, const uint16_t* svh, int P) {
    GemvArgs ga = {};
    ga.x = A;
    ga.x_ld = a_ld;
    ga.tr = tr;
    ga.tn = (int)(n / 16);
    ga.suh = suh;
    ga.S = S;
    ga.sonb = S > 1 ? sonb : nullptr;
    ga.svh = svh;
    ga.out = C;
    ga.out_ld = c_ld;
    ga.P = P;
    ga.nblk = (int)(k / 128);
    ga.a_div = 1;
    return ga;
}

int launch_gemv(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const uint32_t* tr, int64_t n, int K, void* C,
                int64_t c_ld, bool f32, const uint16_t* suh, int S, const int32_t* sonb, const uint16_t* svh,
                hipStream_t st) {
    const int strips = (int)(n / 128), nblk = (int)(k / 128);
    const int P = gemv_splits(strips, nblk, m < kGemvMaxRows ? (int)m : kGemvMaxRows);
    // One row: tagged partials, kept in the counter buffer (zero between calls; a timeout reset zeroes it): 4096 x
    // 4096 7.21 -> 6.88 us, 5376 -> 21504 20.6 -> 19.2 us. With more rows the last split would poll and clear every
    // row's words itself; those calls keep the arrival counters.
    const bool tagged = m == 1;
    Workspace ws;
    int rc = tagged ? workspace(0, (size_t)strips * P * 128, st, &ws)
                    : workspace((size_t)strips * P * kGemvMaxRows * 128 * sizeof(float), (size_t)strips, st, &ws);
    if (rc) return rc;
    GemvArgs ga = gemv_args(A, a_ld, k, tr, n, C, c_ld, suh, S, sonb, svh, P);
    if (tagged) {
        ga.tag = reinterpret_cast<uint32_t*>(ws.counters);
        ga.status = ws.status;
        ga.spin_max = spin_limit();
    } else {
        ga.part = reinterpret_cast<float*>(ws.scratch);
        ga.cnt = ws.counters;
    }
    return gemv_chunks(ga, m, K, f32, strips, 1, st);
}

// ------------------------------------------------------------------------------------------------ allocation-free
// The decode GEMV of exl3_gemm with its split-K partials and arrival counters in a fixed device array instead of the
// library workspace, for callers that cannot allocate (code under HIP graph capture, serving loops). The array lives
// as long as the process, one copy per device; every call on a device shares it (calls that overlap race).
constexpr size_t kNoAllocPartBytes = 16u << 20;              // split-K partials: strips x P x 8 rows x 128 fp32
constexpr size_t kNoAllocCounters = 16384;                   // arrival counters: one per 128-column strip
static __device__ __align__(256) char scratch[kNoAllocPartBytes + kNoAllocCounters * sizeof(int)];

namespace {
std::mutex g_scratch_mu;
char* g_scratch_dev[64];                                      // device address of `scratch`, per device

__global__ void zero_counters_kernel(int* c, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) c[i] = 0;
}
}  // namespace

// Device address of this device's `scratch` (looked up once per device with that device current); the first call
// on a device also clears the counters on `st` (the kernels leave them at zero after every call).
static int noalloc_scratch(hipStream_t st, char** out) {
    int dev = 0;
    EXL3_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail(EXL3_ERR_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        char* p = nullptr;
        EXL3_CHECK_HIP(hipGetSymbolAddress(reinterpret_cast<void**>(&p), HIP_SYMBOL(scratch)));
        hipLaunchKernelGGL(zero_counters_kernel, dim3(64), dim3(256), 0, st,
                           reinterpret_cast<int*>(p + kNoAllocPartBytes), (int)kNoAllocCounters);
        EXL3_CHECK_HIP(hipGetLastError());
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return EXL3_OK;
}

// ------------------------------------------------------------------------------------------------ multi-matrix
// Weighted slot sum of exl3_mgemm: C[t, e] = sum over the token's slots j in order of w[j] * y[j, e] (fp32; skipped
// slots add nothing). Grid (ceil(m n / 256), tokens).
template <bool F32>
__global__ __launch_bounds__(256) void mgemm_sum_kernel(const float* __restrict__ y, int64_t mn,
                                                        const int64_t* __restrict__ idx, int64_t qmin, int64_t qmax,
                                                        int nmat, const uint16_t* __restrict__ w, int per_tok,
                                                        void* __restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int t = blockIdx.y;
    if (e >= mn) return;
    float v = 0.f;
    for (int j0 = 0; j0 < per_tok; j0 += 8) {
        float yv[8], wv[8];
        bool ok[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {                 // every load of a group issued before the first add
            const int jj = t * per_tok + (j0 + i < per_tok ? j0 + i : per_tok - 1);
            ok[i] = j0 + i < per_tok && mgemm_matrix(idx, jj, qmin, qmax, nmat) >= 0;
            yv[i] = y[(int64_t)jj * mn + e];
            wv[i] = h2f(w[jj]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v += ok[i] ? wv[i] * yv[i] : 0.f;
    }
    if (F32) reinterpret_cast<float*>(out)[(int64_t)t * mn + e] = v;
    else reinterpret_cast<uint16_t*>(out)[(int64_t)t * mn + e] = f2h(v);
}

}  // namespace exl3

using namespace exl3;

extern "C" {

int exl3_reconstruct(const int16_t* trellis, int64_t k, int64_t n_total, int K, int cb, int64_t n_offset,
                     int64_t n_slice, uint16_t* out, int64_t out_ld, void* stream) {
    if (cb != 2) return fail(EXL3_ERR_UNSUPPORTED, "exl3_reconstruct: codebook %d not supported (mul1 = 2 only)", cb);
    if (K < 1 || K > 8) return fail(EXL3_ERR_UNSUPPORTED, "exl3_reconstruct: K=%d not in 1..8", K);
    EXL3_CHECK_ARG(trellis && out, "exl3_reconstruct: null pointer");
    EXL3_CHECK_ARG(k > 0 && k % 16 == 0 && n_total % 16 == 0, "exl3_reconstruct: k=%lld n=%lld must be multiples of 16",
                   (long long)k, (long long)n_total);
    EXL3_CHECK_ARG(n_offset % 128 == 0 && n_slice % 128 == 0 && n_offset >= 0 && n_slice >= 0 &&
                       n_offset + n_slice <= n_total,
                   "exl3_reconstruct: slice [%lld, +%lld) of %lld must be 128-aligned and in range",
                   (long long)n_offset, (long long)n_slice, (long long)n_total);
    EXL3_CHECK_ARG(out_ld >= n_slice && out_ld % 8 == 0 && aligned(out, 16),
                   "exl3_reconstruct: output must be 16-byte aligned with a row stride that is a multiple of 8");
    EXL3_CHECK_ARG(aligned(trellis, 4), "exl3_reconstruct: trellis must be 4-byte aligned");
    if (n_slice == 0) return EXL3_OK;
    hipStream_t st = (hipStream_t)stream;
    const uint32_t* tr = reinterpret_cast<const uint32_t*>(trellis);
    dim3 grid((unsigned)(n_slice / 128), (unsigned)(k / 16));
    const int tn = (int)(n_total / 16), n0t = (int)(n_offset / 16);
    typedef void (*rfn)(const uint32_t*, int, int, uint16_t*, int64_t);
    static const rfn fns[8] = {reconstruct_kernel<1>, reconstruct_kernel<2>, reconstruct_kernel<3>,
                               reconstruct_kernel<4>, reconstruct_kernel<5>, reconstruct_kernel<6>,
                               reconstruct_kernel<7>, reconstruct_kernel<8>};
    EXL3_LAUNCH("reconstruct", fns[K - 1], grid, dim3(64), 0, st, tr, tn, n0t, out, out_ld);
    return EXL3_OK;
}

int exl3_reconstruct_had_slice(const int16_t* trellis, int64_t k, int64_t n_total, int K, int cb, const uint16_t* suh,
                               const uint16_t* svh, int64_t n_offset, int64_t n_slice, uint16_t* out, int64_t out_ld,
                               void* stream) {
    if (cb != 2)
        return fail(EXL3_ERR_UNSUPPORTED, "exl3_reconstruct_had_slice: codebook %d not supported (mul1 = 2 only)", cb);
    if (K < 1 || K > 8) return fail(EXL3_ERR_UNSUPPORTED, "exl3_reconstruct_had_slice: K=%d not in 1..8", K);
    EXL3_CHECK_ARG(trellis && suh && svh && out, "exl3_reconstruct_had_slice: null pointer");
    EXL3_CHECK_ARG(k > 0 && k % 128 == 0 && n_total % 128 == 0,
                   "exl3_reconstruct_had_slice: k=%lld and n=%lld must be multiples of 128", (long long)k,
                   (long long)n_total);
    EXL3_CHECK_ARG(n_offset % 128 == 0 && n_slice % 128 == 0 && n_offset >= 0 && n_slice >= 0 &&
                       n_offset + n_slice <= n_total,
                   "exl3_reconstruct_had_slice: slice [%lld, +%lld) of %lld must be 128-aligned and in range",
                   (long long)n_offset, (long long)n_slice, (long long)n_total);
    EXL3_CHECK_ARG(out_ld >= n_slice, "exl3_reconstruct_had_slice: output row stride below the slice width");
    EXL3_CHECK_ARG(aligned(trellis, 4), "exl3_reconstruct_had_slice: trellis must be 4-byte aligned");
    EXL3_CHECK_ARG(k / 128 <= 65535 && n_slice / 128 <= 65535, "exl3_reconstruct_had_slice: shape too large");
    if (n_slice == 0) return EXL3_OK;
    hipStream_t st = (hipStream_t)stream;
    typedef void (*rfn)(const uint32_t*, int, int, const uint16_t*, const uint16_t*, uint16_t*, int64_t);
    static const rfn fns[8] = {reconstruct_had_kernel<1>, reconstruct_had_kernel<2>, reconstruct_had_kernel<3>,
                               reconstruct_had_kernel<4>, reconstruct_had_kernel<5>, reconstruct_had_kernel<6>,
                               reconstruct_had_kernel<7>, reconstruct_had_kernel<8>};
    EXL3_LAUNCH("reconstruct_had", fns[K - 1], dim3((unsigned)(n_slice / 128), (unsigned)(k / 128)), dim3(256), 0, st,
                reinterpret_cast<const uint32_t*>(trellis), (int)(n_total / 16), (int)(n_offset / 16), suh, svh, out,
                out_ld);
    return EXL3_OK;
}

int exl3_had_r_128(const void* in, int64_t in_ld, void* out, int64_t out_ld, int64_t rows, int64_t cols, int dtype,
                   const uint16_t* pre, const uint16_t* post, float scale, void* stream) {
    EXL3_CHECK_ARG(in && out, "exl3_had_r_128: null pointer");
    EXL3_CHECK_ARG(dtype == EXL3_F16 || dtype == EXL3_F32, "exl3_had_r_128: dtype must be fp16 or fp32");
    EXL3_CHECK_ARG(rows >= 0 && cols % 128 == 0 && in_ld >= cols && out_ld >= cols,
                   "exl3_had_r_128: cols=%lld must be a multiple of 128 and row strides >= cols", (long long)cols);
    if (rows == 0 || cols == 0) return EXL3_OK;
    EXL3_CHECK_ARG(rows <= 0x7FFFFFFF && cols / 128 <= 65535, "exl3_had_r_128: shape too large");
    dim3 grid((unsigned)rows, (unsigned)(cols / 128));
    float r = scale * kRsqrt128;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == EXL3_F16)
        EXL3_LAUNCH("had_r_128", had_kernel<true>, grid, dim3(64), 0, st, in, in_ld, out, out_ld, pre, post, r);
    else
        EXL3_LAUNCH("had_r_128", had_kernel<false>, grid, dim3(64), 0, st, in, in_ld, out, out_ld, pre, post, r);
    return EXL3_OK;
}

int exl3_linear_sharded(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const int16_t* B, int64_t n, int K,
                        void* C, int64_t c_ld, int c_dtype, const uint16_t* suh, int64_t n_shards,
                        const int32_t* shard_of_nb, const uint16_t* svh, int cb, void* stream) {
    if (cb != 2) return fail(EXL3_ERR_UNSUPPORTED, "exl3_gemm: codebook %d not supported (mul1 = 2 only)", cb);
    if (K < 1 || K > 8) return fail(EXL3_ERR_UNSUPPORTED, "exl3_gemm: K=%d not in 1..8", K);
    EXL3_CHECK_ARG(c_dtype == EXL3_F16 || c_dtype == EXL3_F32, "exl3_gemm: C must be fp16 or fp32");
    EXL3_CHECK_ARG(m >= 0 && k > 0 && n > 0 && k % 128 == 0 && n % 128 == 0,
                   "exl3_gemm: k=%lld and n=%lld must be positive multiples of 128", (long long)k, (long long)n);
    EXL3_CHECK_ARG(a_ld >= k && c_ld >= n, "exl3_gemm: row strides must cover k / n");
    EXL3_CHECK_ARG(n_shards >= 1 && n_shards <= 64, "exl3_linear_sharded: n_shards=%lld not in 1..64",
                   (long long)n_shards);
    EXL3_CHECK_ARG(n_shards == 1 || shard_of_nb, "exl3_linear_sharded: shard_of_nb required for several shards");
    if (m == 0) return EXL3_OK;
    EXL3_CHECK_ARG(A && B && C && suh && svh, "exl3_gemm: null pointer");
    EXL3_CHECK_ARG(aligned(B, 4), "exl3_gemm: trellis must be 4-byte aligned");
    EXL3_CHECK_ARG(n / 128 <= 65535, "exl3_gemm: n too large");
    EXL3_CHECK_ARG(k / 16 * (n / 16) * 8 * (int64_t)(K > 0 ? K : 8) < (1LL << 32),
                   "exl3_gemm: trellis of %lld x %lld at K=%d exceeds 2^32 words", (long long)k, (long long)n, K);
    const uint32_t* tr = reinterpret_cast<const uint32_t*>(B);
    const int S = (int)n_shards;
    if (m >= env_int("EXL3MI_MFMA_MIN_ROWS", kLinearMfmaMinRows))
        return launch_linear_mfma(A, a_ld, m, k, tr, n, K, C, c_ld, c_dtype == EXL3_F32, suh, S, shard_of_nb, svh,
                                  (hipStream_t)stream);
    return launch_gemv(A, a_ld, m, k, tr, n, K, C, c_ld, c_dtype == EXL3_F32, suh, S, shard_of_nb, svh,
                       (hipStream_t)stream);
}

int exl3_gemm(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const int16_t* B, int64_t n, int K, void* C,
              int64_t c_ld, int c_dtype, const uint16_t* suh, uint16_t* A_had, const uint16_t* svh, int cb,
              void* stream) {
    (void)A_had;
    return exl3_linear_sharded(A, a_ld, m, k, B, n, K, C, c_ld, c_dtype, suh, 1, nullptr, svh, cb, stream);
}

int exl3_gemm_noalloc(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const int16_t* B, int64_t n, int K,
                      void* C, int64_t c_ld, int c_dtype, const uint16_t* suh, const uint16_t* svh, int cb,
                      void* stream) {
    if (cb != 2) return fail(EXL3_ERR_UNSUPPORTED, "exl3_gemm_noalloc: codebook %d not supported (mul1 = 2 only)", cb);
    if (K < 1 || K > 8) return fail(EXL3_ERR_UNSUPPORTED, "exl3_gemm_noalloc: K=%d not in 1..8", K);
    EXL3_CHECK_ARG(c_dtype == EXL3_F16 || c_dtype == EXL3_F32, "exl3_gemm_noalloc: C must be fp16 or fp32");
    EXL3_CHECK_ARG(m >= 0 && m <= kGemvMaxRows, "exl3_gemm_noalloc: m=%lld rows, at most %d", (long long)m,
                   kGemvMaxRows);
    EXL3_CHECK_ARG(k > 0 && n > 0 && k % 128 == 0 && n % 128 == 0,
                   "exl3_gemm_noalloc: k=%lld and n=%lld must be positive multiples of 128", (long long)k,
                   (long long)n);
    EXL3_CHECK_ARG(a_ld >= k && c_ld >= n, "exl3_gemm_noalloc: row strides must cover k / n");
    if (m == 0) return EXL3_OK;
    EXL3_CHECK_ARG(A && B && C && suh && svh, "exl3_gemm_noalloc: null pointer");
    EXL3_CHECK_ARG(aligned(B, 4), "exl3_gemm_noalloc: trellis must be 4-byte aligned");
    EXL3_CHECK_ARG(k / 16 * (n / 16) * 8 * (int64_t)K < (1LL << 32),
                   "exl3_gemm_noalloc: trellis of %lld x %lld at K=%d exceeds 2^32 words", (long long)k,
                   (long long)n, K);
    const int64_t strips = n / 128;
    EXL3_CHECK_ARG(strips <= (int64_t)kNoAllocCounters, "exl3_gemm_noalloc: n=%lld exceeds the %zu columns of the "
                   "fixed scratch", (long long)n, kNoAllocCounters * 128);
    const int P = gemv_splits((int)strips, (int)(k / 128), (int)m);
    const size_t part = (size_t)strips * P * kGemvMaxRows * 128 * sizeof(float);
    EXL3_CHECK_ARG(part <= kNoAllocPartBytes, "exl3_gemm_noalloc: %zu bytes of split-K partials needed, the fixed "
                   "scratch holds %zu", part, kNoAllocPartBytes);
    hipStream_t st = (hipStream_t)stream;
    char* sc = nullptr;
    const int rc = noalloc_scratch(st, &sc);
    if (rc) return rc;
    GemvArgs ga = gemv_args(A, a_ld, k, reinterpret_cast<const uint32_t*>(B), n, C, c_ld, suh, 1, nullptr, svh, P);
    ga.part = reinterpret_cast<float*>(sc);
    ga.cnt = reinterpret_cast<int*>(sc + kNoAllocPartBytes);
    return gemv_chunks(ga, m, K, c_dtype == EXL3_F32, (int)strips, 1, st, false);
}

int exl3_mgemm(const uint16_t* A, int64_t a_batches, int64_t m, int64_t k, const int64_t* B_ptrs,
               const int64_t* suh_ptrs, const int64_t* svh_ptrs, int64_t num_mats, int64_t n, int K, int cb,
               const int64_t* indices, int64_t slots, const uint16_t* weights, int64_t num_tokens, int64_t min_index,
               int64_t max_index, void* C, int c_dtype, void* stream) {
    if (cb != 2) return fail(EXL3_ERR_UNSUPPORTED, "exl3_mgemm: codebook %d not supported (mul1 = 2 only)", cb);
    if (K < 1 || K > 8) return fail(EXL3_ERR_UNSUPPORTED, "exl3_mgemm: K=%d not in 1..8", K);
    EXL3_CHECK_ARG(c_dtype == EXL3_F16 || c_dtype == EXL3_F32, "exl3_mgemm: C must be fp16 or fp32");
    EXL3_CHECK_ARG(m >= 0 && k > 0 && n > 0 && k % 128 == 0 && n % 128 == 0,
                   "exl3_mgemm: k=%lld and n=%lld must be positive multiples of 128", (long long)k, (long long)n);
    EXL3_CHECK_ARG(num_mats >= 1 && num_mats <= 0x7FFFFFFF, "exl3_mgemm: num_mats=%lld", (long long)num_mats);
    EXL3_CHECK_ARG(slots >= 0 && slots <= 65535, "exl3_mgemm: slots=%lld not in 0..65535", (long long)slots);
    EXL3_CHECK_ARG(indices || slots <= num_mats, "exl3_mgemm: without indices slot j uses matrix j (slots <= num_mats)");
    const bool weighted = weights != nullptr;
    EXL3_CHECK_ARG(!weighted || (num_tokens >= 1 && num_tokens <= 65535 && slots % num_tokens == 0),
                   "exl3_mgemm: weighted sum needs 1 <= num_tokens <= 65535 dividing slots (%lld)", (long long)slots);
    const int64_t per_tok = num_tokens >= 1 && slots % num_tokens == 0 ? slots / num_tokens : 0;
    EXL3_CHECK_ARG(a_batches == 1 || a_batches == slots || (per_tok > 0 && a_batches == num_tokens),
                   "exl3_mgemm: a_batches=%lld must be 1, slots (%lld) or num_tokens (%lld)", (long long)a_batches,
                   (long long)slots, (long long)num_tokens);
    EXL3_CHECK_ARG(min_index < 0 || max_index > min_index, "exl3_mgemm: max_index must exceed min_index");
    EXL3_CHECK_ARG(n / 128 <= 65535, "exl3_mgemm: n too large");
    EXL3_CHECK_ARG(k / 16 * (n / 16) * 8 * (int64_t)K < (1LL << 32),
                   "exl3_mgemm: trellis of %lld x %lld at K=%d exceeds 2^32 words", (long long)k, (long long)n, K);
    if (m == 0 || (slots == 0 && !weighted)) return EXL3_OK;
    EXL3_CHECK_ARG(A && B_ptrs && suh_ptrs && svh_ptrs && C, "exl3_mgemm: null pointer");
    const bool f32 = c_dtype == EXL3_F32;
    hipStream_t st = (hipStream_t)stream;
    const int strips = (int)(n / 128), nblk = (int)(k / 128);
    const int64_t units = (int64_t)strips * (slots > 0 ? slots : 1);          // strips of every slot
    const int P = gemv_splits(units < (1 << 30) ? (int)units : (1 << 30), nblk,
                              m < kGemvMaxRows ? (int)m : kGemvMaxRows);
    const size_t part_bytes = carve_size((size_t)slots * strips * P * kGemvMaxRows * 128, sizeof(float));
    const size_t y_bytes = weighted ? carve_size((size_t)slots * m * n, sizeof(float)) : 0;
    Workspace ws;
    int rc = workspace(part_bytes + y_bytes, (size_t)(slots > 0 ? slots : 1) * strips, st, &ws);
    if (rc) return rc;
    Carve cv{ws.scratch, ws.scratch_bytes};
    float* part = cv.take<float>((size_t)slots * strips * P * kGemvMaxRows * 128);
    float* y = weighted ? cv.take<float>((size_t)slots * m * n) : nullptr;
    if (!part || (weighted && !y)) return fail(EXL3_ERR_HIP, "exl3_mgemm: workspace carve failed");
    if (slots > 0) {
        GemvArgs ga = {};
        ga.x = A;
        ga.x_ld = k;
        ga.tn = (int)(n / 16);
        ga.S = 1;
        ga.out = weighted ? (void*)y : C;
        ga.out_ld = n;
        ga.part = part;
        ga.cnt = ws.counters;
        ga.P = P;
        ga.nblk = nblk;
        ga.trp = B_ptrs;
        ga.suhp = suh_ptrs;
        ga.svhp = svh_ptrs;
        ga.idx = indices;
        ga.nmat = (int)num_mats;
        ga.qmin = min_index;
        ga.qmax = max_index;
        ga.a_div = a_batches == 1 || a_batches == slots ? 1 : (int)per_tok;
        ga.x_bs = a_batches == 1 ? 0 : m * k;
        ga.out_bs = m * n;
        rc = gemv_chunks(ga, m, K, weighted || f32, strips, (int)slots, st);
        if (rc) return rc;
    }
    if (weighted) {
        const int64_t mn = m * n;
        EXL3_CHECK_ARG((mn + 255) / 256 <= 0x7FFFFFFF, "exl3_mgemm: m * n too large");
        const dim3 grid((unsigned)((mn + 255) / 256), (unsigned)num_tokens);
        if (f32)
            EXL3_LAUNCH("mgemm_sum", mgemm_sum_kernel<true>, grid, dim3(256), 0, st, y, mn, indices, min_index,
                        max_index, (int)num_mats, weights, (int)per_tok, C);
        else
            EXL3_LAUNCH("mgemm_sum", mgemm_sum_kernel<false>, grid, dim3(256), 0, st, y, mn, indices, min_index,
                        max_index, (int)num_mats, weights, (int)per_tok, C);
    }
    return EXL3_OK;
}

}  // extern "C"
