// Expert-sorted ragged grouped GEMM on fp16 MFMA for experts with many rows (prefill chunks).
//
// Rows (token, expert pairs) are grouped by expert and cut into blocks of MB rows. Per layer call:
//   pairs_had   transformed gate / up inputs of every block row: xh[pair][proj] = fp16(H128(fp16(x * suh)) / sqrt(128))
//   gateup      workgroup per (block, 128-column block of I), full H: each wave decodes two gate and two up tile
//               columns per 32-k step straight into MFMA B fragments (the codebook affine is folded: B holds h values,
//               the epilogue applies c1 * acc + c2 * rowsum(A)), then the fused activation / down-input epilogue
//   down        workgroup per (block, 128-column block of H), full I, epilogue Hadamard * svh_d * w and the combine
// Workgroup ids are laid out so that the column blocks of one expert block run on one XCD (shared L2 for A).
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
__global__ __launch_bounds__(256) void pairs_had_kernel(MoeArgs a) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int blk = blockIdx.x, kb = blockIdx.y;
    const ItemDesc* d = a.blocks + blk;
    const int cnt = d->cnt;
    if (cnt == 0) return;
    const int p0 = d->p0;
    for (int i = wave; i < 2 * cnt; i += 4) {
        const int row = i >> 1, proj = i & 1;
        const int tok = a.pair_tok[p0 + row];
        const uint16_t* suh = reinterpret_cast<const uint16_t*>(d->tab[3 * proj + 1]) + kb * 128;
        _Float16* dst = a.xh + ((size_t)(p0 + row) * 2 + proj) * a.H + kb * 128;
        had_in_block(a.x + (int64_t)tok * a.x_ld + kb * 128, suh, dst, lane);
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
// One wave accumulates T tile columns (tile column t from projection t / (T / NP)) over all 32-k steps for RG row
// groups of A (NP activation streams, one per projection). Weight words run two steps ahead (ring of 3), A fragments
// one step ahead (ring of 2); the loop is unrolled 6x so every buffer is consumed where it was filled, and each
// step issues A(s+1) before W(s+2) so waiting for a step's data never waits for a later prefetch.
template <int K, int T, int NP, int RG>
struct MfmaLoop {
    static constexpr int NW = FragCfg<K>::NW;
    static constexpr int TPP = T / NP;          // tile columns per projection
    const uint32_t* wbase[T];                   // tile (tile-row lane >> 5, column) of step 0, per tile column
    size_t wstep;                               // words between consecutive steps (two tile-rows)
    const _Float16* abase[NP][RG];              // A row pointer (with this lane's k offset) per projection / group
    int nsteps;
    FragCfg<K> cfg;

    __device__ __forceinline__ void load_w(uint32_t (&W)[T][NW], int s) const {
        const size_t off = (size_t)(s < nsteps ? s : nsteps - 1) * wstep;
#pragma unroll
        for (int t = 0; t < T; ++t) frag_load<K>(wbase[t] + off, cfg, W[t]);
        __builtin_amdgcn_sched_barrier(0);
    }
    __device__ __forceinline__ void load_a(h8_t (&A)[NP][RG], int s) const {
        const int ss = (s < nsteps ? s : nsteps - 1) * 32;
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) A[p][rg] = *reinterpret_cast<const h8_t*>(abase[p][rg] + ss);
        __builtin_amdgcn_sched_barrier(0);
    }
    __device__ __forceinline__ void compute(uint32_t (&W)[T][NW], const h8_t (&A)[NP][RG], f4_t (&acc)[T][RG],
                                            float (&rs)[NP][RG]) const {
        h8_t bf[T];
#pragma unroll
        for (int t = 0; t < T; ++t) bf[t] = frag_finish<K>(W[t], cfg.sh);
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                float sv = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) sv += (float)A[p][rg][j];
                rs[p][rg] += sv;
#pragma unroll
                for (int u = 0; u < TPP; ++u)
                    acc[p * TPP + u][rg] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(A[p][rg], bf[p * TPP + u], acc[p * TPP + u][rg], 0, 0, 0);
            }
    }
    __device__ __forceinline__ void run(f4_t (&acc)[T][RG], float (&rs)[NP][RG]) const {
        uint32_t W0[T][NW], W1[T][NW], W2[T][NW];
        h8_t A0[NP][RG], A1[NP][RG];
        load_a(A0, 0);
        load_w(W0, 0);
        load_w(W1, 1);
        int s = 0;
        for (; s + 6 <= nsteps; s += 6) {
            load_a(A1, s + 1); load_w(W2, s + 2); compute(W0, A0, acc, rs);
            load_a(A0, s + 2); load_w(W0, s + 3); compute(W1, A1, acc, rs);
            load_a(A1, s + 3); load_w(W1, s + 4); compute(W2, A0, acc, rs);
            load_a(A0, s + 4); load_w(W2, s + 5); compute(W0, A1, acc, rs);
            load_a(A1, s + 5); load_w(W0, s + 6); compute(W1, A0, acc, rs);
            load_a(A0, s + 6); load_w(W1, s + 7); compute(W2, A1, acc, rs);
        }
        // tail (< 6 steps): W0 / W1 hold steps s, s + 1 and A0 holds step s
        if (s < nsteps) { load_a(A1, s + 1); load_w(W2, s + 2); compute(W0, A0, acc, rs); }
        if (s + 1 < nsteps) { load_a(A0, s + 2); load_w(W0, s + 3); compute(W1, A1, acc, rs); }
        if (s + 2 < nsteps) { load_a(A1, s + 3); load_w(W1, s + 4); compute(W2, A0, acc, rs); }
        if (s + 3 < nsteps) { load_a(A0, s + 4); load_w(W2, s + 5); compute(W0, A1, acc, rs); }
        if (s + 4 < nsteps) { load_a(A1, s + 5); compute(W1, A0, acc, rs); }
    }
};

// ------------------------------------------------------------------------------------------------ gate | up
template <int K, int MB>
__global__ __launch_bounds__(256) void gateup_mfma_kernel(MoeArgs a) {
    extern __shared__ float smem[];
    constexpr int RG = MB / 16;
    float* C = smem;                         // [2][MB][128]
    float* rsum = smem + 2 * MB * 128;       // [2][MB]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nbI = a.I / 128;
    int blk, nb;
    xcd_map(nbI, blk, nb);
    if (blk >= a.max_blocks) return;
    const ItemDesc* d = a.blocks + blk;
    const int cnt = d->cnt;
    if (cnt == 0) return;
    const int p0 = d->p0;
    const int tn = a.I / 16;
    const uint32_t* trp[2] = {reinterpret_cast<const uint32_t*>(d->tab[0]),
                              reinterpret_cast<const uint32_t*>(d->tab[3])};
    const uint8_t* kmp[2] = {reinterpret_cast<const uint8_t*>(d->km[0]), reinterpret_cast<const uint8_t*>(d->km[2])};
    const int32_t* wop[2] = {reinterpret_cast<const int32_t*>(d->km[1]), reinterpret_cast<const int32_t*>(d->km[3])};
    const int ct0 = nb * 8 + 2 * wave;
    const _Float16* arow[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        int r = 16 * rg + (lane & 15);
        r = r < cnt ? r : cnt - 1;
        arow[rg] = a.xh + (size_t)(p0 + r) * 2 * a.H + 8 * (lane >> 4);
    }
    f4_t acc[4][RG];
    float rs[2][RG];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) acc[t][rg] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) rs[p][rg] = 0.f;

    const int nsteps = a.H / 32;
    if (K > 0) {
        constexpr int KL = K > 0 ? K : 1;
        MfmaLoop<KL, 4, 2, RG> L;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            L.wbase[t] = trp[t >> 1] + ((size_t)(lane >> 5) * tn + ct0 + (t & 1)) * (8 * KL);
        L.wstep = (size_t)2 * tn * 8 * KL;
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) L.abase[p][rg] = arow[rg] + (size_t)p * a.H;
        L.nsteps = nsteps;
        frag_setup<KL>(lane, L.cfg);
        L.run(acc, rs);
    }
    for (int s = 0; K == 0 && s < nsteps; ++s) {
        const int tr = 2 * s + (lane >> 5);
        h8_t bf[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int p = t >> 1, col = ct0 + (t & 1);
            {
                const int tile = tr * tn + col;
                bf[t] = frag_decode_k(trp[p] + ldg(wop[p] + tile), ldg(kmp[p] + tile), lane);
            }
        }
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const h8_t av = *reinterpret_cast<const h8_t*>(arow[rg] + (size_t)p * a.H + 32 * s);
                float sv = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) sv += (float)av[j];
                rs[p][rg] += sv;
                acc[2 * p][rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bf[2 * p], acc[2 * p][rg], 0, 0, 0);
                acc[2 * p + 1][rg] =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bf[2 * p + 1], acc[2 * p + 1][rg], 0, 0, 0);
            }
        }
    }

    // row sums: lanes L, L ^ 16, L ^ 32, L ^ 48 hold the four k-groups of row L & 15
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            float v = rs[p][rg];
            v += lane_xor<16>(v, lane);
            v += lane_xor<32>(v, lane);
            if (wave == 0 && lane < 16) rsum[p * MB + 16 * rg + lane] = v;
        }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int p = t >> 1, col = (2 * wave + (t & 1)) * 16 + (lane & 15);
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int i = 0; i < 4; ++i) C[(p * MB + 16 * rg + 4 * (lane >> 4) + i) * 128 + col] = acc[t][rg][i];
    }
    __syncthreads();

    const uint16_t* svg = reinterpret_cast<const uint16_t*>(d->tab[2]) + nb * 128;
    const uint16_t* svu = reinterpret_cast<const uint16_t*>(d->tab[5]) + nb * 128;
    const uint16_t* sud = reinterpret_cast<const uint16_t*>(d->tab[7]) + nb * 128;
    for (int m = wave; m < cnt; m += 4) {
        const float sg = kMul1C2 * rsum[m], su = kMul1C2 * rsum[MB + m];
        float g0 = kMul1C1 * C[m * 128 + lane] + sg, g1 = kMul1C1 * C[m * 128 + lane + 64] + sg;
        float u0 = kMul1C1 * C[(MB + m) * 128 + lane] + su, u1 = kMul1C1 * C[(MB + m) * 128 + lane + 64] + su;
        fwht128_wave(g0, g1, lane);
        fwht128_wave(u0, u1, lane);
        g0 = (float)(_Float16)(g0 * kRsqrt128 * h2f(ldg(svg + lane)));
        g1 = (float)(_Float16)(g1 * kRsqrt128 * h2f(ldg(svg + lane + 64)));
        u0 = (float)(_Float16)(u0 * kRsqrt128 * h2f(ldg(svu + lane)));
        u1 = (float)(_Float16)(u1 * kRsqrt128 * h2f(ldg(svu + lane + 64)));
        float a0 = (float)(_Float16)act_mul_dev(g0, u0, a.act, a.limit);
        float a1 = (float)(_Float16)act_mul_dev(g1, u1, a.act, a.limit);
        a0 = (float)(_Float16)(a0 * h2f(ldg(sud + lane)));
        a1 = (float)(_Float16)(a1 * h2f(ldg(sud + lane + 64)));
        fwht128_wave(a0, a1, lane);
        uint16_t* dst = a.abuf + (size_t)(p0 + m) * a.I + nb * 128;
        dst[lane] = f2h(a0 * kRsqrt128);
        dst[lane + 64] = f2h(a1 * kRsqrt128);
    }
}

// ------------------------------------------------------------------------------------------------ down
template <int K, int MB>
__global__ __launch_bounds__(256) void down_mfma_kernel(MoeArgs a) {
    extern __shared__ float smem[];
    constexpr int RG = MB / 16;
    float* C = smem;                         // [MB][128]
    float* rsum = smem + MB * 128;           // [MB]
    __shared__ int s_comb[MB];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nbH = a.H / 128;
    int blk, nb;
    xcd_map(nbH, blk, nb);
    if (blk >= a.max_blocks) return;
    const ItemDesc* d = a.blocks + blk;
    const int cnt = d->cnt;
    if (cnt == 0) return;
    const int p0 = d->p0;
    const int tn = a.H / 16;
    const uint32_t* trd = reinterpret_cast<const uint32_t*>(d->tab[6]);
    const uint8_t* kmd = reinterpret_cast<const uint8_t*>(d->km[4]);
    const int32_t* wod = reinterpret_cast<const int32_t*>(d->km[5]);
    const int ct0 = nb * 8 + 2 * wave;
    const uint16_t* arow[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        int r = 16 * rg + (lane & 15);
        r = r < cnt ? r : cnt - 1;
        arow[rg] = a.abuf + (size_t)(p0 + r) * a.I + 8 * (lane >> 4);
    }
    f4_t acc[2][RG];
    float rs[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        acc[0][rg] = acc[1][rg] = f4_t{0.f, 0.f, 0.f, 0.f};
        rs[rg] = 0.f;
    }
    const int nsteps = a.I / 32;
    if (K > 0) {
        constexpr int KL = K > 0 ? K : 1;
        MfmaLoop<KL, 2, 1, RG> L;
#pragma unroll
        for (int t = 0; t < 2; ++t) L.wbase[t] = trd + ((size_t)(lane >> 5) * tn + ct0 + t) * (8 * KL);
        L.wstep = (size_t)2 * tn * 8 * KL;
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) L.abase[0][rg] = reinterpret_cast<const _Float16*>(arow[rg]);
        L.nsteps = nsteps;
        frag_setup<KL>(lane, L.cfg);
        f4_t acc1[2][RG];
        float rs1[1][RG];
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            acc1[0][rg] = acc[0][rg];
            acc1[1][rg] = acc[1][rg];
            rs1[0][rg] = rs[rg];
        }
        L.run(acc1, rs1);
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            acc[0][rg] = acc1[0][rg];
            acc[1][rg] = acc1[1][rg];
            rs[rg] = rs1[0][rg];
        }
    }
    for (int s = 0; K == 0 && s < nsteps; ++s) {
        const int tr = 2 * s + (lane >> 5);
        h8_t bf[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int col = ct0 + t;
            {
                const int tile = tr * tn + col;
                bf[t] = frag_decode_k(trd + ldg(wod + tile), ldg(kmd + tile), lane);
            }
        }
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            const h8_t av = *reinterpret_cast<const h8_t*>(arow[rg] + 32 * s);
            float sv = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) sv += (float)av[j];
            rs[rg] += sv;
            acc[0][rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bf[0], acc[0][rg], 0, 0, 0);
            acc[1][rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bf[1], acc[1][rg], 0, 0, 0);
        }
    }
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        float v = rs[rg];
        v += lane_xor<16>(v, lane);
        v += lane_xor<32>(v, lane);
        if (wave == 0 && lane < 16) rsum[16 * rg + lane] = v;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int col = (2 * wave + t) * 16 + (lane & 15);
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int i = 0; i < 4; ++i) C[(16 * rg + 4 * (lane >> 4) + i) * 128 + col] = acc[t][rg][i];
    }
    __syncthreads();

    const uint16_t* svd = reinterpret_cast<const uint16_t*>(d->tab[8]) + nb * 128;
    for (int m = wave; m < cnt; m += 4) {
        const float sx = kMul1C2 * rsum[m];
        float v0 = kMul1C1 * C[m * 128 + lane] + sx, v1 = kMul1C1 * C[m * 128 + lane + 64] + sx;
        fwht128_wave(v0, v1, lane);
        const float w = a.pair_w[p0 + m];
        float* dst = a.y + (size_t)(p0 + m) * a.H + nb * 128;
        splitk_store(dst + lane, v0 * kRsqrt128 * h2f(ldg(svd + lane)) * w);
        splitk_store(dst + lane + 64, v1 * kRsqrt128 * h2f(ldg(svd + lane + 64)) * w);
    }
    // combine: count rows into their tokens, finish tokens whose slots are all in
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int nbH_ = nbH;
    for (int m = threadIdx.x; m < cnt; m += 256) {
        const int t = a.pair_tok[p0 + m];
        const int old = __hip_atomic_fetch_add(&a.cnt_tok[(size_t)t * nbH_ + nb], 1, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
        s_comb[m] = (old == a.tok_nvalid[t] - 1) ? t : -1;
    }
    __syncthreads();
    for (int m = wave; m < cnt; m += 4)
        if (s_comb[m] >= 0) combine_token(a, s_comb[m], nb, lane);
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

template <int MB>
static mfma_fn pick_gu(int K) {
    switch (K) {
        case 0: return gateup_mfma_kernel<0, MB>;
        case 1: return gateup_mfma_kernel<1, MB>;
        case 2: return gateup_mfma_kernel<2, MB>;
        case 3: return gateup_mfma_kernel<3, MB>;
        case 4: return gateup_mfma_kernel<4, MB>;
        case 5: return gateup_mfma_kernel<5, MB>;
        case 6: return gateup_mfma_kernel<6, MB>;
        case 7: return gateup_mfma_kernel<7, MB>;
        default: return gateup_mfma_kernel<8, MB>;
    }
}

template <int MB>
static mfma_fn pick_dn(int K) {
    switch (K) {
        case 0: return down_mfma_kernel<0, MB>;
        case 1: return down_mfma_kernel<1, MB>;
        case 2: return down_mfma_kernel<2, MB>;
        case 3: return down_mfma_kernel<3, MB>;
        case 4: return down_mfma_kernel<4, MB>;
        case 5: return down_mfma_kernel<5, MB>;
        case 6: return down_mfma_kernel<6, MB>;
        case 7: return down_mfma_kernel<7, MB>;
        default: return down_mfma_kernel<8, MB>;
    }
}

int mfma_lds_gu(int MB) { return (2 * MB * 128 + 2 * MB) * (int)sizeof(float); }
int mfma_lds_dn(int MB) { return (MB * 128 + MB) * (int)sizeof(float); }

int launch_moe_mfma_gateup(const MoeArgs& a, hipStream_t st) {
    constexpr int MB = kMfmaRows;
    const int nxb = (a.max_blocks + 7) / 8 * 8;
    EXL3_LAUNCH("moe_pairs_had", pairs_had_kernel, dim3(a.max_blocks, a.H / 128), dim3(256), 0, st, a);
    mfma_fn fn = pick_gu<MB>(a.Kg);
    const int lds = mfma_lds_gu(MB);
    EXL3_CHECK_HIP(set_max_lds((const void*)fn, lds));
    EXL3_LAUNCH("moe_gateup_mfma", fn, dim3(nxb * (a.I / 128)), dim3(256), lds, st, a);
    return EXL3_OK;
}

int launch_moe_mfma_down(const MoeArgs& a, hipStream_t st) {
    constexpr int MB = kMfmaRows;
    const int nxb = (a.max_blocks + 7) / 8 * 8;
    mfma_fn fn = pick_dn<MB>(a.Kd);
    const int lds = mfma_lds_dn(MB);
    EXL3_CHECK_HIP(set_max_lds((const void*)fn, lds));
    EXL3_LAUNCH("moe_down_mfma", fn, dim3(nxb * (a.H / 128)), dim3(256), lds, st, a);
    return EXL3_OK;
}

}  // namespace exl3
