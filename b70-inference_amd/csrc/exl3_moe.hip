// Grouped EXL3 MoE on gfx950: routing tables, decode GEMV path (gate|up + fused activation epilogue, down, combine),
// and the softmax/top-k router.
//
// Per layer call (all on the caller's stream, no host synchronisation):
//   align    one workgroup: expert histogram -> pairs grouped by expert, the inverse map pair_of[token, slot], and
//            "items" = (expert, first pair, <= MR rows) work units; the GEMV grids are sized for the worst case and
//            surplus workgroups exit (the reference's max_act launch, glm/xpu/csrc/exl3_moe.n128.sycl:691-734, 1380-1439)
//   gateup   workgroup per (item, 128-column block of I, k-split of H): gate and up strips (2 waves each), split-K
//            handoff, and in the last workgroup: Hadamard * svh -> fp16 g, u -> fp16 act(g, u) -> * suh_d -> Hadamard
//            -> fp16 down input (the reference's GateUpKernel epilogue, exl3_moe.n128.sycl:253-271)
//   down     workgroup per (item, 128-column block of H, k-split of I): Hadamard * svh_d * w -> y[pair] fp32
//   combine  out[t] = sum over slots in order of y[pair_of[t, slot]] (deterministic, exl3_moe.n128.sycl:385-410)
// Experts with more than MR rows (prefill) are handled by the MFMA grouped GEMM (exl3_mfma.hip).
#include "exl3_device.h"
#include "exl3_gemv.h"
#include "exl3_moe.h"
#include "exl3_moe_dev.h"
#include "exl3_runtime.h"

namespace exl3 {

// ================================================================================================ align
// Exclusive scan of n ints in LDS by a 1024-thread workgroup. Returns the total. Up to one value per thread: shuffle
// scans within the waves, then over the wave totals (three barriers); more: each thread scans a contiguous run.
__device__ int block_scan_exclusive(int* a, int n, int* tmp /* [1024] */) {
    const int t = threadIdx.x, T = blockDim.x;
    if (n <= T) {
        const int lane = t & 63, wv = t >> 6, nw = T >> 6;
        const int v = t < n ? a[t] : 0;
        int x = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int y = __shfl_up(x, d);
            if (lane >= d) x += y;
        }
        if (lane == 63) tmp[wv] = x;
        __syncthreads();
        if (t < 64) {
            int w = t < nw ? tmp[t] : 0;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int y = __shfl_up(w, d);
                if (t >= d) w += y;
            }
            tmp[64 + t] = w;
        }
        __syncthreads();
        if (t < n) a[t] = (wv > 0 ? tmp[64 + wv - 1] : 0) + x - v;
        const int total = tmp[64 + nw - 1];
        __syncthreads();
        return total;
    }
    const int per = (n + T - 1) / T;
    const int lo = t * per, hi = min(n, lo + per);
    int s = 0;
    for (int i = lo; i < hi; ++i) s += a[i];
    tmp[t] = s;
    __syncthreads();
    for (int d = 1; d < T; d <<= 1) {
        int v = t >= d ? tmp[t - d] : 0;
        __syncthreads();
        tmp[t] += v;
        __syncthreads();
    }
    int run = tmp[t] - s;   // exclusive prefix of this thread's run
    const int total = tmp[T - 1];
    for (int i = lo; i < hi; ++i) {
        int v = a[i];
        a[i] = run;
        run += v;
    }
    __syncthreads();
    return total;
}

// Workgroup barrier for LDS only: every LDS access before it has completed and is visible after it, while global
// stores keep draining (a kernel whose global writes are read only by later kernels need not wait for them here).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Exclusive scans of three LDS arrays of n <= blockDim.x ints at once (shuffle scans within the waves; every wave
// then adds up the wave totals below it itself, so two barriers in all); tot[] gets the totals.
__device__ void block_scan3(int* a, int* b, int* c, int n, int* tmp /* [48] */, int (&tot)[3]) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6, nw = blockDim.x >> 6;
    int* arr[3] = {a, b, c};
    int v[3], x[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) x[i] = v[i] = t < n ? arr[i][t] : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        int y[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) y[i] = __shfl_up(x[i], d);
#pragma unroll
        for (int i = 0; i < 3; ++i) x[i] += lane >= d ? y[i] : 0;
    }
    if (lane == 63)
#pragma unroll
        for (int i = 0; i < 3; ++i) tmp[16 * i + wv] = x[i];
    lds_barrier();
    int u[3][16];                      // every wave total read first (one LDS round trip), then summed
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int w = 0; w < 16; ++w) u[i][w] = w < nw ? tmp[16 * i + w] : 0;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        int below = 0, all = 0;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            below += w < wv ? u[i][w] : 0;
            all += u[i][w];
        }
        if (t < n) arr[i][t] = below + x[i] - v[i];
        tot[i] = all;
    }
    lds_barrier();
}

// Experts, weights and tokens of pairs i0 + k * stride, k < B (-1 / 0 past np or for an invalid id), every load
// issued before any is used: indices are clamped instead of branched on, so a batch costs one memory round trip. The
// (token, slot) of each pair is carried from the first by the stride's quotient and remainder (integer division is
// a long VALU sequence here: three per call instead of two per pair).
template <int B>
__device__ __forceinline__ void load_pairs(const RouteArgs& r, int i0, int stride, int np, int (&e)[B],
                                           float (&w)[B], int (&tk)[B]) {
    int jq[B];
    {
        int tok = i0 / r.slots, j = i0 - tok * r.slots;
        const int dq = stride / r.slots, dr = stride - dq * r.slots;
#pragma unroll
        for (int k = 0; k < B; ++k) {
            tk[k] = tok;
            jq[k] = j;
            tok += dq;
            j += dr;
            if (j >= r.slots) {
                j -= r.slots;
                ++tok;
            }
        }
    }
    const int tlast = (np - 1) / r.slots, jlast = np - 1 - tlast * r.slots;   // the clamp target, pair np - 1
    int v[B];
    float wv[B];
    if (r.topk > 0) {
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const bool in = i0 + k * stride < np;
            const int tok = in ? tk[k] : tlast, j = in ? jq[k] : jlast, jj = j < r.topk ? j : r.topk - 1;
            v[k] = ldg(r.ids + tok * r.topk + jj);
            wv[k] = ldg(r.tw + tok * r.topk + jj);
        }
    } else {
#pragma unroll
        for (int k = 0; k < B; ++k) {
            v[k] = 0;
            wv[k] = 1.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < B; ++k) {
        const bool in = i0 + k * stride < np;
        const int j = jq[k];
        const int ek = j < r.topk ? v[k] : r.shared;
        e[k] = in && ek >= 0 && ek < r.E ? ek : -1;
        w[k] = j < r.topk ? wv[k] : 1.0f;
    }
}

// An item or block descriptor's head and table entries in 16-byte stores (the tab and km fields are contiguous from a
// 16-byte boundary), so that one thread writing many descriptors issues half as many scattered stores.
__device__ __forceinline__ void write_desc(ItemDesc& d, int e, int p0, int cnt, const int64_t (&tb)[9],
                                           const int64_t (&km)[6]) {
    static_assert(offsetof(ItemDesc, tab) % 16 == 0 && offsetof(ItemDesc, km) == offsetof(ItemDesc, tab) + 72,
                  "descriptor table layout");
    typedef int64_t i64x2_t __attribute__((ext_vector_type(2)));
    typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
    int64_t v[15];
#pragma unroll
    for (int i = 0; i < 9; ++i) v[i] = tb[i];
#pragma unroll
    for (int i = 0; i < 6; ++i) v[9 + i] = km[i];
    *reinterpret_cast<i32x4_t*>(&d) = i32x4_t{e, p0, cnt, 0};
    i64x2_t* q = reinterpret_cast<i64x2_t*>(d.tab);
#pragma unroll
    for (int j = 0; j < 7; ++j) q[j] = i64x2_t{v[2 * j], v[2 * j + 1]};
    d.km[5] = v[14];
}

// The memory round trips are the kernel's cost, so with held pairs (np <= 8 * 1024) every load is issued at the start:
// the thread's pairs (kept in registers for the scatter) and its first expert's table entries; the tokens' valid
// slots are counted in LDS with the experts' rows instead of reloading each token's slots, and the counting atomics'
// values (a pair's rank within its expert) place the pairs, so the scatter needs no second atomic. The barriers order
// LDS only: the tables written here are read by later kernels, so their stores drain behind the rest of the kernel.
__global__ __launch_bounds__(1024) void align_kernel(RouteArgs r) {
    extern __shared__ int sm[];
    int* cnt = sm;                 // [E]
    int* start = sm + r.E;         // [E]
    int* fill = sm + 2 * r.E;      // [E]
    int* nch = sm + 3 * r.E;       // [E] GEMV items of the expert, then their first index
    int* nbl = sm + 4 * r.E;       // [E] MFMA blocks of the expert, then their first index
    int* tmp = sm + 5 * r.E;       // [1024]
    int* tokn = sm + 5 * r.E + 1024;   // [M] valid slots per token (held pairs)
    int* stok = tokn + r.M;            // [M * slots] x 3: pair_tok, pair_w, pair_e in sorted order (staged)
    float* sw = reinterpret_cast<float*>(stok + r.M * r.slots);
    int* se = stok + 2 * r.M * r.slots;
    __shared__ int s_cls[3];
    const int t = threadIdx.x, T = blockDim.x;
    if (t < 3) s_cls[t] = 0;
    const int np = r.M * r.slots;
    const int mr = r.MR > 0 ? r.MR : 1;   // MR == 0: every expert with rows is an MFMA expert (no GEMV items)
    int hev[8], htk[8];
    float hwv[8];
    if (r.held) load_pairs<8>(r, t, T, np, hev, hwv, htk);
    // this thread's first expert's table entries (index clamped: unconditional loads)
    int64_t tb0[9], km0[6];
    {
        const int ec = t < r.E ? t : r.E - 1;
#pragma unroll
        for (int i = 0; i < 9; ++i) tb0[i] = r.items ? ldg(r.tables + (int64_t)i * r.E + ec) : 0;
#pragma unroll
        for (int i = 0; i < 6; ++i) km0[i] = r.items && r.kmaps ? ldg(r.kmaps + (int64_t)i * r.E + ec) : 0;
    }
    for (int e = t; e < r.E; e += T) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    if (r.held)
        for (int m = t; m < r.M; m += T) tokn[m] = 0;
    lds_barrier();
    int hrk[8];                        // held pairs: each pair's rank within its expert (the counting atomic's value)
    if (r.held) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (hev[k] >= 0) {
                hrk[k] = atomicAdd(&cnt[hev[k]], 1);
                atomicAdd(&tokn[htk[k]], 1);
            }
    } else {
        for (int i0 = t; i0 < np; i0 += 8 * T) {
            int ev[8], tk[8];
            float wv[8];
            load_pairs<8>(r, i0, T, np, ev, wv, tk);
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (ev[k] >= 0) atomicAdd(&cnt[ev[k]], 1);
        }
    }
    lds_barrier();
    for (int e = t; e < r.E; e += T) {
        const int c = cnt[e];
        const bool big = r.use_mfma && c > r.MR;
        start[e] = c;
        nch[e] = big ? 0 : (c + mr - 1) / mr;
        nbl[e] = big ? (c + r.MB - 1) / r.MB : 0;
    }
    lds_barrier();
    int nvalid, nitems, nblocks;
    if (r.E <= T) {
        int tot[3];
        block_scan3(start, nch, nbl, r.E, tmp, tot);
        nvalid = tot[0];
        nitems = tot[1];
        nblocks = tot[2];
    } else {
        nvalid = block_scan_exclusive(start, r.E, tmp);
        nitems = block_scan_exclusive(nch, r.E, tmp);
        nblocks = block_scan_exclusive(nbl, r.E, tmp);
    }
    if (r.pair_e)
        for (int i = nvalid + t; i < np; i += T) r.pair_e[i] = -1;
    for (int e = t; e < r.E; e += T) {
        const int c = cnt[e];
        if (r.counts) r.counts[e] = c;
        if (!r.items || c == 0) continue;
        const bool big = r.use_mfma && c > r.MR;
        // the expert's table entries, loaded once for all of its blocks / items (the first expert's at the start)
        int64_t tb[9], km[6];
#pragma unroll
        for (int i = 0; i < 9; ++i) tb[i] = e == t ? tb0[i] : ldg(r.tables + (int64_t)i * r.E + e);
        if (r.kmaps) {
#pragma unroll
            for (int i = 0; i < 6; ++i) km[i] = e == t ? km0[i] : ldg(r.kmaps + (int64_t)i * r.E + e);
        } else {
#pragma unroll
            for (int i = 0; i < 6; ++i) km[i] = 0;
        }
        for (int q = 0, b = nbl[e]; big && q * r.MB < c; ++q, ++b) {
            ItemDesc& d = r.blocks[b];
            const int dc = min(r.MB, c - q * r.MB);
            write_desc(d, e, start[e] + q * r.MB, dc, tb, km);
            if (r.cls_list) {
                const int cl = mfma_row_class(dc);
                r.cls_list[cl * r.max_blocks + atomicAdd(&s_cls[cl], 1)] = b;
            }
        }
        for (int q = 0, it = nch[e]; !big && q * mr < c; ++q, ++it) {
            write_desc(r.items[it], e, start[e] + q * mr, min(mr, c - q * mr), tb, km);
        }
    }
    if (r.items)
        for (int it = nitems + t; it < r.max_items; it += T) r.items[it].cnt = 0;
    if (r.blocks)
        for (int b = nblocks + t; b < r.max_blocks; b += T) r.blocks[b].cnt = 0;
    if (t == 0 && r.n_items) r.n_items[0] = nitems;
    lds_barrier();
    if (t < 3 && r.cls_cnt) r.cls_cnt[t] = s_cls[t];
    if (r.tok_nvalid) {
        for (int tok = t; tok < r.M; tok += T) {
            int nv = 0;
            if (r.held) {
                nv = tokn[tok];
            } else {
                for (int j0 = 0; j0 < r.slots; j0 += 8) {
                    int ev[8], tk[8];
                    float wv[8];
                    load_pairs<8>(r, tok * r.slots + j0, 1, tok * r.slots + r.slots, ev, wv, tk);
#pragma unroll
                    for (int k = 0; k < 8; ++k) nv += ev[k] >= 0;
                }
            }
            r.tok_nvalid[tok] = nv;
            if (nv == 0) {
                for (int c = 0; c < r.H; ++c) {
                    if (r.out_f32) reinterpret_cast<float*>(r.out)[(int64_t)tok * r.out_ld + c] = 0.f;
                    else reinterpret_cast<uint16_t*>(r.out)[(int64_t)tok * r.out_ld + c] = 0;
                }
            }
        }
    }
    lds_barrier();
    for (int i0 = t; i0 < np; i0 += 8 * T) {
        int ev[8], tk[8];
        float wv[8];
        if (r.held) {                  // i0 == t: the pairs loaded at the start
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                ev[k] = hev[k];
                wv[k] = hwv[k];
                tk[k] = htk[k];
            }
        } else {
            load_pairs<8>(r, i0, T, np, ev, wv, tk);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = i0 + k * T;
            if (i >= np) break;
            const int tok = tk[k], e = ev[k];
            if (e >= 0) {
                const int f = r.held ? hrk[k] : atomicAdd(&fill[e], 1);
                const int pos = start[e] + f;
                const float wt = wv[k];
                if (r.staged) {
                    stok[pos] = tok;
                    sw[pos] = wt;
                    se[pos] = e;
                } else {
                    r.pair_tok[pos] = tok;
                    r.pair_w[pos] = wt;
                    if (r.pair_e) r.pair_e[pos] = e;
                }
                r.pair_of[i] = pos;
                if (r.items && !(r.use_mfma && cnt[e] > r.MR)) {
                    ItemDesc& d = r.items[nch[e] + f / mr];
                    d.tok[f % mr] = tok;
                    d.w[f % mr] = wt;
                }
            } else {
                r.pair_of[i] = -1;
            }
        }
    }
    if (r.staged) {                    // the sorted pairs out of LDS, coalesced
        lds_barrier();
        for (int q = t; q < nvalid; q += T) {
            r.pair_tok[q] = stok[q];
            r.pair_w[q] = sw[q];
            if (r.pair_e) r.pair_e[q] = se[q];
        }
    }
}

// Same tables for at most kAlignSmall pairs, one thread per pair: a pair's place in the expert-sorted order is the
// number of valid pairs with a lower expert plus those of its own expert earlier in flat order; item and block indices
// are counts of chunk leaders (a pair whose index within its expert is a multiple of MR, or of MB for MFMA blocks)
// placed at or before it. No scan over E, a handful of barriers.
constexpr int kAlignSmall = 256;

__global__ __launch_bounds__(kAlignSmall) void align_small_kernel(RouteArgs r) {
    __shared__ int s_e[kAlignSmall], s_pos[kAlignSmall];
    __shared__ uint8_t s_lead[kAlignSmall], s_blead[kAlignSmall];
    __shared__ int s_cls[3];
    const int t = threadIdx.x;
    if (t < 3) s_cls[t] = 0;
    const int np = r.M * r.slots;
    const int mr = r.MR > 0 ? r.MR : 1;   // MR == 0: every expert with rows is an MFMA expert (no GEMV items)
    int e = -1, tok = 0;
    float wt = 0.f;
    if (t < np) {
        tok = t / r.slots;
        const int j = t - tok * r.slots;
        e = j < r.topk ? ldg(r.ids + tok * r.topk + j) : r.shared;
        if (e >= r.E) e = -1;
        wt = j < r.topk ? ldg(r.tw + tok * r.topk + j) : 1.0f;
    }
    s_e[t] = e;
    __syncthreads();
    int below = 0, before = 0, cnt = 0;
    if (e >= 0)
        for (int q = 0; q < np; ++q) {
            const int eq = s_e[q];
            below += eq >= 0 && eq < e;
            before += eq == e && q < t;
            cnt += eq == e;
        }
    const int pos = below + before;
    const bool big = e >= 0 && r.use_mfma && cnt > r.MR;
    const bool lead = e >= 0 && !big && before % mr == 0;
    const bool blead = big && before % r.MB == 0;
    s_pos[t] = e >= 0 ? pos : 0x7FFFFFFF;
    s_lead[t] = lead;
    s_blead[t] = blead;
    const int nvalid = __syncthreads_count(e >= 0);
    int nitems = 0, nblocks = 0, item = 0, block = 0;
    for (int q = 0; q < np; ++q) {
        const int pq = s_pos[q];
        if (s_lead[q]) {
            ++nitems;
            item += pq <= pos;
        }
        if (s_blead[q]) {
            ++nblocks;
            block += pq <= pos;
        }
    }
    --item;
    --block;
    if (t < np) {
        if (e >= 0) {
            r.pair_tok[pos] = tok;
            r.pair_w[pos] = wt;
            r.pair_of[t] = pos;
            if (r.pair_e) r.pair_e[pos] = e;
        } else {
            r.pair_of[t] = -1;
        }
        if (r.pair_e && t >= nvalid) r.pair_e[t] = -1;
    }
    if (r.items) {
        if (lead) {
            ItemDesc& d = r.items[item];
            d.e = e;
            d.p0 = pos;
            d.cnt = min(mr, cnt - before);
            for (int i = 0; i < 9; ++i) d.tab[i] = ldg(r.tables + (int64_t)i * r.E + e);
            for (int i = 0; i < 6; ++i) d.km[i] = r.kmaps ? ldg(r.kmaps + (int64_t)i * r.E + e) : 0;
        }
        if (e >= 0 && !big) {
            ItemDesc& d = r.items[item];
            d.tok[before % mr] = tok;
            d.w[before % mr] = wt;
        }
        for (int it = nitems + t; it < r.max_items; it += kAlignSmall) r.items[it].cnt = 0;
        if (t == 0 && r.n_items) r.n_items[0] = nitems;
    }
    if (r.blocks) {
        if (blead) {
            ItemDesc& d = r.blocks[block];
            d.e = e;
            d.p0 = pos;
            d.cnt = min(r.MB, cnt - before);
            for (int i = 0; i < 9; ++i) d.tab[i] = ldg(r.tables + (int64_t)i * r.E + e);
            for (int i = 0; i < 6; ++i) d.km[i] = r.kmaps ? ldg(r.kmaps + (int64_t)i * r.E + e) : 0;
            if (r.cls_list) {
                const int cl = mfma_row_class(d.cnt);
                r.cls_list[cl * r.max_blocks + atomicAdd(&s_cls[cl], 1)] = block;
            }
        }
        for (int b = nblocks + t; b < r.max_blocks; b += kAlignSmall) r.blocks[b].cnt = 0;
    }
    __syncthreads();
    if (t < 3 && r.cls_cnt) r.cls_cnt[t] = s_cls[t];
    if (r.counts)
        for (int x = t; x < r.E; x += kAlignSmall) {
            int c = 0;
            for (int q = 0; q < np; ++q) c += s_e[q] == x;
            r.counts[x] = c;
        }
    if (r.tok_nvalid)
        for (int tk = t; tk < r.M; tk += kAlignSmall) {
            int nv = 0;
            for (int j = 0; j < r.slots; ++j) nv += s_e[tk * r.slots + j] >= 0;
            r.tok_nvalid[tk] = nv;
            if (nv == 0)
                for (int c = 0; c < r.H; ++c) {
                    if (r.out_f32) reinterpret_cast<float*>(r.out)[(int64_t)tk * r.out_ld + c] = 0.f;
                    else reinterpret_cast<uint16_t*>(r.out)[(int64_t)tk * r.out_ld + c] = 0;
                }
        }
}

// ================================================================================================ gate | up
template <int K, int MR, bool PL = false>
__global__ __launch_bounds__(256) void gateup_kernel(MoeArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][MR][kGemvKBMax * 128];
    __shared__ float red[4][MR][2][64];
    __shared__ float bsum[2][MR][kGemvKBMax];
    __shared__ int s_last;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nbI = a.I / 128;
    const int item = blockIdx.x / nbI, nb = blockIdx.x - item * nbI, p = blockIdx.y;
    const ItemDesc* d = a.items + item;
    const int cnt = d->cnt;
    if (cnt == 0) return;
    const int p0 = d->p0;
    const int b0 = (int)((int64_t)p * a.nblk_h / a.P_gu), b1 = (int)((int64_t)(p + 1) * a.nblk_h / a.P_gu);
    const int kb = b1 - b0;
    const int proj = wave >> 1, half = wave & 1;
    const uint32_t* tr = reinterpret_cast<const uint32_t*>(d->tab[3 * proj]);
    const int tn = a.I / 16;
    constexpr int KL = K > 0 ? K : 1;
    const size_t rs = (size_t)a.gu_tn * (8 * KL);
    const uint32_t* sp = tr + (size_t)nb * (64 * KL) + (size_t)b0 * 8 * rs;
    // phase 1: both projections' input transforms for the item's rows. The wave's first JB blocks of x and signs are
    // loaded before the weight prefetch (unconditional loads at clamped addresses, prefetch without a branch:
    // half < 8 <= kb * 8), so their transforms wait for nothing issued after them; later blocks load afterwards.
    const int nbm = 2 * MR * kb;
    auto block_ptrs = [&](int i, const uint16_t*& xp, const uint16_t*& sq) {
        const int proj = i / (MR * kb), rem = i - proj * MR * kb, m = rem / kb, b = rem - m * kb;
        const int k0 = (b0 + b) * 128;
        sq = reinterpret_cast<const uint16_t*>(d->tab[3 * proj + 1]) + k0;
        xp = a.x + (int64_t)d->tok[m < cnt ? m : 0] * a.x_ld + k0;
    };
    constexpr int JB = 2;
    HadIn hv[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int i = wave + 4 * j;
        const uint16_t *xp, *sq;
        block_ptrs(i < nbm ? i : nbm - 1, xp, sq);
        hv[j] = had_in_load(xp, sq, lane);
    }
    StripRing<KL, 3> ring;
    if (K > 0) strip_prefetch<KL, 3, false, PL>(sp, rs, half, kb * 8, 2, lane, ring);
    auto finish = [&](int i, const HadIn& h) {
        const int proj = i / (MR * kb), rem = i - proj * MR * kb, m = rem / kb, b = rem - m * kb;
        const float s = had_in_finish(h, m < cnt, &xs[proj][m][b * 128], lane);
        if (lane == 0) bsum[proj][m][b] = s;
    };
#pragma unroll
    for (int j = 0; j < JB; ++j)
        if (wave + 4 * j < nbm) finish(wave + 4 * j, hv[j]);
    for (int i = wave + 4 * JB; i < nbm; i += 4) {
        const uint16_t *xp, *sq;
        block_ptrs(i, xp, sq);
        finish(i, had_in_load(xp, sq, lane));
    }
    __syncthreads();

    // phase 2: waves 0, 1 stream the gate strip, waves 2, 3 the up strip (alternating tile-rows)
    float acc[MR][2];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m][0] = acc[m][1] = 0.f;
    if (K > 0) {
        strip_gemv_run<KL, MR, 3, PL>(sp, rs, half, kb * 8, 2, lane, &xs[proj][0][0], kGemvKBMax * 128, acc, ring);
    } else {
        const uint8_t* km = reinterpret_cast<const uint8_t*>(d->km[2 * proj]);
        const int32_t* wo = reinterpret_cast<const int32_t*>(d->km[2 * proj + 1]);
        strip_gemv_mixed<MR>(tr, km, wo, tn, nb * 8, b0 * 8, half, kb * 8, 2, lane, &xs[proj][0][0],
                             kGemvKBMax * 128, acc);
    }

    // phase 3: per projection, fold the two waves, the codebook affine, publish the split's partial
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        red[wave][m][0][lane] = acc[m][0];
        red[wave][m][1][lane] = acc[m][1];
    }
    __syncthreads();
    const int cbase = 16 * (lane >> 3) + (lane & 7);
    const size_t slot = (size_t)item * nbI + nb;
    if (half == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float sx = 0.f;
            for (int b = 0; b < kb; ++b) sx += bsum[proj][m][b];
            float* dst = a.part_gu + (((slot * a.P_gu + p) * 2 + proj) * MR + m) * 128;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float v = red[wave][m][h][lane] + red[wave + 1][m][h][lane];
                splitk_store(dst + cbase + 8 * h, kMul1C1 * v + kMul1C2 * sx);
            }
        }
    }
    if (!splitk_arrive(&a.cnt_gu[slot], a.P_gu, &s_last)) return;

    // epilogue (last workgroup of this item / column block)
    const uint16_t* svg = reinterpret_cast<const uint16_t*>(d->tab[2]) + nb * 128;
    const uint16_t* svu = reinterpret_cast<const uint16_t*>(d->tab[5]) + nb * 128;
    const uint16_t* sud = reinterpret_cast<const uint16_t*>(d->tab[7]) + nb * 128;
    for (int m = wave; m < cnt; m += 4) {
        float g0 = 0.f, g1 = 0.f, u0 = 0.f, u1 = 0.f;
#pragma unroll 4
        for (int pp = 0; pp < a.P_gu; ++pp) {
            const float* q = a.part_gu + ((slot * a.P_gu + pp) * 2) * MR * 128 + m * 128;
            g0 += splitk_load(q + lane);
            g1 += splitk_load(q + lane + 64);
            u0 += splitk_load(q + MR * 128 + lane);
            u1 += splitk_load(q + MR * 128 + lane + 64);
        }
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
    if (threadIdx.x == 0) a.cnt_gu[slot] = 0;
}

// ================================================================================================ down (+ combine)
// The last workgroup of an (item, column block) writes its rows' weighted outputs y, then counts them in per-(token,
// column block) arrival counters; the workgroup that completes a token's slots sums them in slot order into `out`
// (the reference's CombineKernel, fused: no separate launch).
template <int K, int MR, bool PL = false>
__global__ __launch_bounds__(256) void down_kernel(MoeArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[MR][kGemvKBMax * 128];
    __shared__ float red[4][MR][2][64];
    __shared__ float bsum[MR][kGemvKBMax];
    __shared__ int s_last;
    __shared__ int s_comb[MR];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nbH = a.H / 128;
    const int item = blockIdx.x / nbH, nb = blockIdx.x - item * nbH, p = blockIdx.y;
    const ItemDesc* d = a.items + item;
    const int cnt = d->cnt;
    if (cnt == 0) return;
    const int p0 = d->p0;
    const int b0 = (int)((int64_t)p * a.nblk_i / a.P_d), b1 = (int)((int64_t)(p + 1) * a.nblk_i / a.P_d);
    const int kb = b1 - b0;
    const uint32_t* tr = reinterpret_cast<const uint32_t*>(d->tab[6]);
    const int tn = a.H / 16;
    constexpr int KL = K > 0 ? K : 1;
    const size_t rs = (size_t)tn * (8 * KL);
    const uint32_t* sp = tr + (size_t)nb * (64 * KL) + (size_t)b0 * 8 * rs;
    // the wave's first JB input blocks loaded before the weight prefetch (as in gateup_kernel; wave < 8 <= kb * 8)
    const int nbm = MR * kb;
    auto src_of = [&](int i) {
        const int m = i / kb, b = i - m * kb;
        return a.abuf + (size_t)(p0 + (m < cnt ? m : 0)) * a.I + (b0 + b) * 128;
    };
    constexpr int JB = 2;
    uint16_t ca[JB], cb[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int i = wave + 4 * j;
        const uint16_t* src = src_of(i < nbm ? i : nbm - 1);
        ca[j] = ldg(src + lane);
        cb[j] = ldg(src + lane + 64);
    }
    StripRing<KL, 3> ring;
    if (K > 0) strip_prefetch<KL, 3, false, PL>(sp, rs, wave, kb * 8, 4, lane, ring);
    auto put = [&](int i, uint16_t va, uint16_t vb) {
        const int m = i / kb, b = i - m * kb;
        const _Float16 ha = m < cnt ? __builtin_bit_cast(_Float16, va) : (_Float16)0.f;
        const _Float16 hb = m < cnt ? __builtin_bit_cast(_Float16, vb) : (_Float16)0.f;
        xs[m][b * 128 + lane] = ha;
        xs[m][b * 128 + lane + 64] = hb;
        const float s = wave_sum_f32((float)ha + (float)hb);
        if (lane == 0) bsum[m][b] = s;
    };
#pragma unroll
    for (int j = 0; j < JB; ++j)
        if (wave + 4 * j < nbm) put(wave + 4 * j, ca[j], cb[j]);
    for (int i = wave + 4 * JB; i < nbm; i += 4) {
        const uint16_t* src = src_of(i);
        put(i, ldg(src + lane), ldg(src + lane + 64));
    }
    __syncthreads();

    float acc[MR][2];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m][0] = acc[m][1] = 0.f;
    if (K > 0) {
        strip_gemv_run<KL, MR, 3, PL>(sp, rs, wave, kb * 8, 4, lane, &xs[0][0], kGemvKBMax * 128, acc, ring);
    } else {
        const uint8_t* km = reinterpret_cast<const uint8_t*>(d->km[4]);
        const int32_t* wo = reinterpret_cast<const int32_t*>(d->km[5]);
        strip_gemv_mixed<MR>(tr, km, wo, tn, nb * 8, b0 * 8, wave, kb * 8, 4, lane, &xs[0][0], kGemvKBMax * 128,
                             acc);
    }

#pragma unroll
    for (int m = 0; m < MR; ++m) {
        red[wave][m][0][lane] = acc[m][0];
        red[wave][m][1][lane] = acc[m][1];
    }
    __syncthreads();
    const int cbase = 16 * (lane >> 3) + (lane & 7);
    const size_t slot = (size_t)item * nbH + nb;
    if (wave == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float sx = 0.f;
            for (int b = 0; b < kb; ++b) sx += bsum[m][b];
            float* dst = a.part_d + ((slot * a.P_d + p) * MR + m) * 128;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float v = red[0][m][h][lane] + red[1][m][h][lane] + red[2][m][h][lane] + red[3][m][h][lane];
                splitk_store(dst + cbase + 8 * h, kMul1C1 * v + kMul1C2 * sx);
            }
        }
    }
    if (!splitk_arrive(&a.cnt_d[slot], a.P_d, &s_last)) return;

    const uint16_t* svd = reinterpret_cast<const uint16_t*>(d->tab[8]) + nb * 128;
    for (int m = wave; m < cnt; m += 4) {
        float v0 = 0.f, v1 = 0.f;
#pragma unroll 4
        for (int pp = 0; pp < a.P_d; ++pp) {
            const float* q = a.part_d + ((slot * a.P_d + pp) * MR + m) * 128;
            v0 += splitk_load(q + lane);
            v1 += splitk_load(q + lane + 64);
        }
        fwht128_wave(v0, v1, lane);
        const float w = d->w[m];
        float* dst = a.y + (size_t)(p0 + m) * a.H + nb * 128;
        splitk_store(dst + lane, v0 * kRsqrt128 * h2f(ldg(svd + lane)) * w);
        splitk_store(dst + lane + 64, v1 * kRsqrt128 * h2f(ldg(svd + lane + 64)) * w);
    }
    if (threadIdx.x == 0) a.cnt_d[slot] = 0;

    // combine: count this item's rows into their tokens; finish the tokens whose slots are now all in
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int m = 0; m < cnt; ++m) {
            const int t = d->tok[m];
            const int old = __hip_atomic_fetch_add(&a.cnt_tok[(size_t)t * nbH + nb], 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
            s_comb[m] = (old == a.tok_nvalid[t] - 1) ? t : -1;
        }
    }
    __syncthreads();
    for (int m = wave; m < cnt; m += 4)
        if (s_comb[m] >= 0) combine_token(a, s_comb[m], nb, lane);
}

// ================================================================================================ router
// One wave per row (route_row).
template <int V, int SC>
__global__ __launch_bounds__(64) void route_kernel(const float* __restrict__ logits, int64_t ld, int E,
                                                   const float* __restrict__ bias, int k, int flags, float scaling,
                                                   int32_t* __restrict__ ids, float* __restrict__ w) {
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    int id;
    float wt;
    route_row<V, SC>(logits + row * ld, bias, E, k, lane, !(flags & EXL3_ROUTE_BIAS_SELECT_ONLY),
                     (flags & EXL3_ROUTE_RENORM) != 0, scaling, id, wt);
    if (lane < k) {
        ids[row * k + lane] = id;
        w[row * k + lane] = wt;
    }
}

typedef void (*route_fn)(const float*, int64_t, int, const float*, int, int, float, int32_t*, float*);

// route_kernel with the picks ranked by s * mul + b + max(res, -1e30) (route_row's ADJ form).
template <int V, int SC>
__global__ __launch_bounds__(64) void route_adj_kernel(const float* __restrict__ logits, int64_t ld, int E,
                                                       const float* __restrict__ bias, const float* __restrict__ mul,
                                                       const float* __restrict__ res, int k, int flags, float scaling,
                                                       int32_t* __restrict__ ids, float* __restrict__ w) {
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    int id;
    float wt;
    route_row<V, SC, true>(logits + row * ld, bias, E, k, lane, true, (flags & EXL3_ROUTE_RENORM) != 0, scaling, id,
                           wt, mul, res);
    if (lane < k) {
        ids[row * k + lane] = id;
        w[row * k + lane] = wt;
    }
}

// Verify blocks of S rows, one wave per block, rows in order (sqrt-softplus): an expert that an earlier row of the
// block picked ranks by s * mul * (1 + boost) + b instead of s * mul + b (each operation rounded separately), so the
// block reads fewer distinct experts; the weights stay the plain s, renormalised (+1e-20) and scaled (the reference's
// RouteBlock, dsv41/xpu/csrc/dsv_moe_glue.sycl:194-240).
template <int V>
__global__ __launch_bounds__(64) void route_block_kernel(const float* __restrict__ logits, int64_t ld, int E,
                                                         const float* __restrict__ bias, const float* __restrict__ mul,
                                                         int k, int S, float boost, float scaling,
                                                         int32_t* __restrict__ ids, float* __restrict__ w) {
    const int lane = threadIdx.x;
    bool chosen[V];
#pragma unroll
    for (int v = 0; v < V; ++v) chosen[v] = false;
    const float up = 1.0f + boost;
    for (int si = 0; si < S; ++si) {
        const int64_t row = (int64_t)blockIdx.x * S + si;
        float f[V], b[V], m[V], g[V];
        uint32_t key[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int i = lane + 64 * v < E ? lane + 64 * v : E - 1;
            f[v] = ldg(logits + row * ld + i);
            b[v] = bias ? ldg(bias + i) : 0.f;
            m[v] = mul ? ldg(mul + i) : 1.f;
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const float sv = sqrtf(f[v] > 20.f ? f[v] : log1pf(expf(f[v])));
            g[v] = sv;
            float r = __fmul_rn(__fmul_rn(sv, m[v]), chosen[v] ? up : 1.0f);
            if (bias) r = __fadd_rn(r, b[v]);
            key[v] = lane + 64 * v < E ? (r != r ? 1u : float_key(r)) : 0u;
        }
        int id;
        float wt;
        route_select<V, EXL3_SCORE_SQRT_SOFTPLUS>(key, g, 0.f, 1.f, k, lane, true, scaling, id, wt);
        if (lane < k) {
            ids[row * k + lane] = id;
            w[row * k + lane] = wt;
        }
        for (int j = 0; j < k; ++j) {                 // the row's picks join the block's chosen experts
            const int pid = __builtin_amdgcn_readlane(id, j);
#pragma unroll
            for (int v = 0; v < V; ++v)
                if (pid >= 0 && pid == lane + 64 * v) chosen[v] = true;
        }
    }
}

typedef void (*route_block_fn)(const float*, int64_t, int, const float*, const float*, int, int, float, float,
                               int32_t*, float*);

typedef void (*route_adj_fn)(const float*, int64_t, int, const float*, const float*, const float*, int, int, float,
                             int32_t*, float*);

template <int SC>
static route_adj_fn route_adj_pick(int64_t E) {
    return E <= 64 ? route_adj_kernel<1, SC> : E <= 128 ? route_adj_kernel<2, SC> : E <= 256 ? route_adj_kernel<4, SC>
         : E <= 512 ? route_adj_kernel<8, SC> : E <= 1024 ? route_adj_kernel<16, SC> : route_adj_kernel<32, SC>;
}

template <int SC>
static route_fn route_pick(int64_t E) {
    return E <= 64 ? route_kernel<1, SC> : E <= 128 ? route_kernel<2, SC> : E <= 256 ? route_kernel<4, SC>
         : E <= 512 ? route_kernel<8, SC> : E <= 1024 ? route_kernel<16, SC> : E <= 2048 ? route_kernel<32, SC>
         : E <= 4096 ? route_kernel<64, SC> : route_kernel<128, SC>;
}

// Router logits, W [H][E] (the reference's gate_tensor): workgroup of 16 waves per (64 expert columns, MR rows).
// Lane 8 r + c of wave q reads W rows h = h0 + 8 i + r (h0: the wave's 1/16 of H, 128 rows per batch) at columns
// 8c .. 8c + 7 with one 16-byte load each, the batch's x values staged in LDS; products accumulate in fp32 per lane,
// then over r (lane shuffles) and over the 16 waves (LDS, in wave order).
constexpr int kRtWaves = 16;
template <int MR>
__global__ __launch_bounds__(1024) void router_cols_kernel(const uint16_t* __restrict__ x, int64_t x_ld, int M, int H,
                                                           const uint16_t* __restrict__ W, int64_t w_ld, int E,
                                                           int round16, float* __restrict__ out, int64_t out_ld) {
    __shared__ _Float16 xs[kRtWaves][MR][128];
    __shared__ float red[kRtWaves][MR][64];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane >> 3, c = lane & 7;
    const int e0 = blockIdx.x * 64, m0 = blockIdx.y * MR;
    const int ce = e0 + 8 * c < E ? e0 + 8 * c : E - 8;          // in-bounds chunk (results past E unused)
    const int hw = H / kRtWaves, h0 = wave * hw;                 // hw: a multiple of 8
    float acc[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[m][j] = 0.f;
    for (int hb = 0; hb < hw; hb += 128) {
        // stage x[m0 + m][h0 + hb + (0 .. 127)] (zeros past the wave's rows or past M)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int row = m0 + m < M ? m0 + m : M - 1;
            const int hh = hb + 2 * lane;
            const uint32_t v = ldg(reinterpret_cast<const uint32_t*>(x + (int64_t)row * x_ld + h0 + (hh < hw ? hh : 0)));
            const bool ok = m0 + m < M && hh < hw;
            *reinterpret_cast<uint32_t*>(&xs[wave][m][2 * lane]) = ok ? v : 0u;
        }
        __syncthreads();
        u32x4_t wv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int hh = hb + 8 * i + r;
            wv[i] = ldg(reinterpret_cast<const u32x4_t*>(W + (int64_t)(h0 + (hh < hw ? hh : hw - 1)) * w_ld + ce));
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const h8_t wh = __builtin_bit_cast(h8_t, wv[i]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float xv = (float)xs[wave][m][8 * i + r];
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[m][j] = fmaf(xv, (float)wh[j], acc[m][j]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float v = acc[m][j];
            v += __shfl_xor(v, 8);
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            acc[m][j] = v;
        }
    if (r == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int j = 0; j < 8; ++j) red[wave][m][8 * c + j] = acc[m][j];
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < MR * 64) {
        const int m = t >> 6, col = t & 63;
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < kRtWaves; ++q) v += red[q][m][col];
        if (m0 + m < M && e0 + col < E) out[(int64_t)(m0 + m) * out_ld + e0 + col] = round16 ? (float)(_Float16)v : v;
    }
}

// Router logits, W [E][H] (a linear layer's weight): wave per expert, lanes along H with 16-byte loads of W and of
// the MR x rows, fp32 products, one wave sum per row.
template <int MR>
__global__ __launch_bounds__(256) void router_rows_kernel(const uint16_t* __restrict__ x, int64_t x_ld, int M, int H,
                                                          const uint16_t* __restrict__ W, int64_t w_ld, int E,
                                                          int round16, float* __restrict__ out, int64_t out_ld) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = blockIdx.x * 4 + wave, m0 = blockIdx.y * MR;
    if (e >= E) return;
    const uint16_t* wr = W + (int64_t)e * w_ld;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    for (int h0 = 8 * lane; h0 < H; h0 += 4 * 512) {
        u32x4_t wv[4], xv[4][MR];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int h = h0 + 512 * i < H ? h0 + 512 * i : h0;      // unconditional (repeats h0, unused)
            wv[i] = ldg(reinterpret_cast<const u32x4_t*>(wr + h));
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const int row = m0 + m < M ? m0 + m : M - 1;
                xv[i][m] = ldg(reinterpret_cast<const u32x4_t*>(x + (int64_t)row * x_ld + h));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (h0 + 512 * i >= H) break;
            const h8_t wh = __builtin_bit_cast(h8_t, wv[i]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const h8_t xh = __builtin_bit_cast(h8_t, xv[i][m]);
                float t = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) t = fmaf((float)xh[j], (float)wh[j], t);
                acc[m] += t;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const float v = wave_sum_f32(acc[m]);
        if (lane == 0 && m0 + m < M) out[(int64_t)(m0 + m) * out_ld + e] = round16 ? (float)(_Float16)v : v;
    }
}

// ================================================================================================ act_mul
template <bool F16>
__global__ __launch_bounds__(256) void act_mul_kernel(const void* __restrict__ x, const void* __restrict__ y,
                                                      uint16_t* __restrict__ z, int64_t n, int act, float L) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float g, u;
    if (F16) {
        g = h2f(reinterpret_cast<const uint16_t*>(x)[i]);
        u = h2f(reinterpret_cast<const uint16_t*>(y)[i]);
    } else {
        g = reinterpret_cast<const float*>(x)[i];
        u = reinterpret_cast<const float*>(y)[i];
    }
    z[i] = f2h(act_mul_dev(g, u, act, L));
}

// ================================================================================================ host
static size_t align_lds_bytes(int E) { return (size_t)(5 * E + 1024) * sizeof(int); }

int launch_align(const RouteArgs& r, hipStream_t st) {
    if ((int64_t)r.M * r.slots <= kAlignSmall) {
        EXL3_LAUNCH("moe_align", align_small_kernel, dim3(1), dim3(kAlignSmall), 0, st, r);
        return EXL3_OK;
    }
    // held pairs when every pair fits the threads' registers and the token counts fit the 64 KB of dynamic LDS
    RouteArgs h = r;
    const size_t lds0 = align_lds_bytes(r.E), ldsh = lds0 + (size_t)r.M * sizeof(int);
    h.held = (int64_t)r.M * r.slots <= 8 * 1024 && ldsh <= 65536;
    const size_t ldss = ldsh + 3 * (size_t)r.M * r.slots * sizeof(int);
    h.staged = h.held && ldss + 256 <= 65536;        // (room for the kernel's static LDS)
    EXL3_LAUNCH("moe_align", align_kernel, dim3(1), dim3(1024), h.staged ? ldss : h.held ? ldsh : lds0, st, h);
    return EXL3_OK;
}

static int moe_splits(int units, int nblk) {
    const int target = env_int("EXL3MI_TARGET_WG", kGemvTargetWG);
    int P = (target + units - 1) / (units > 0 ? units : 1);
    int pmin = (nblk + kGemvKBMax - 1) / kGemvKBMax;
    if (P < pmin) P = pmin;
    if (P > nblk) P = nblk;
    return P < 1 ? 1 : P;
}

typedef void (*moe_fn)(MoeArgs);

// PLANAR4 instantiations exist where the order differs from tile order (D = K / gcd(K, 32) > 1: K = 3, 5, 6, 7)
template <int MR>
static moe_fn pick_gateup(int K, bool pl) {
    if (pl) {
        switch (K) {
            case 3: return gateup_kernel<3, MR, true>;
            case 5: return gateup_kernel<5, MR, true>;
            case 6: return gateup_kernel<6, MR, true>;
            case 7: return gateup_kernel<7, MR, true>;
            default: break;
        }
    }
    switch (K) {
        case 0: return gateup_kernel<0, MR>;
        case 1: return gateup_kernel<1, MR>;
        case 2: return gateup_kernel<2, MR>;
        case 3: return gateup_kernel<3, MR>;
        case 4: return gateup_kernel<4, MR>;
        case 5: return gateup_kernel<5, MR>;
        case 6: return gateup_kernel<6, MR>;
        case 7: return gateup_kernel<7, MR>;
        default: return gateup_kernel<8, MR>;
    }
}

template <int MR>
static moe_fn pick_down(int K, bool pl) {
    if (pl) {
        switch (K) {
            case 3: return down_kernel<3, MR, true>;
            case 5: return down_kernel<5, MR, true>;
            case 6: return down_kernel<6, MR, true>;
            case 7: return down_kernel<7, MR, true>;
            default: break;
        }
    }
    switch (K) {
        case 0: return down_kernel<0, MR>;
        case 1: return down_kernel<1, MR>;
        case 2: return down_kernel<2, MR>;
        case 3: return down_kernel<3, MR>;
        case 4: return down_kernel<4, MR>;
        case 5: return down_kernel<5, MR>;
        case 6: return down_kernel<6, MR>;
        case 7: return down_kernel<7, MR>;
        default: return down_kernel<8, MR>;
    }
}

static moe_fn gateup_select(int K, int MR, bool pl) {
    switch (MR) {
        case 1: return pick_gateup<1>(K, pl);
        case 2: return pick_gateup<2>(K, pl);
        case 4: return pick_gateup<4>(K, pl);
        default: return pick_gateup<8>(K, pl);
    }
}

static moe_fn down_select(int K, int MR, bool pl) {
    switch (MR) {
        case 1: return pick_down<1>(K, pl);
        case 2: return pick_down<2>(K, pl);
        case 4: return pick_down<4>(K, pl);
        default: return pick_down<8>(K, pl);
    }
}

int launch_moe_mfma(const MoeArgs& a, hipStream_t st);          // exl3_mfma.hip
bool moe_fused_ok(const MoeArgs& a);                            // exl3_moe_fused.hip
bool moe_fused_take(const MoeArgs& a);
double moe_expected_items(const MoeArgs& m, int mr);
int moe_fused_path(const MoeArgs& a, hipStream_t st);

// One layer call: align, then GEMV items (experts with <= MR rows) and MFMA blocks (more rows), gate|up before down.
// `a` has every field but the route / workspace ones set.
int moe_decode_path(MoeArgs a, int64_t npairs, hipStream_t st) {
    const int max_items = a.max_items;
    const int nbI = a.I / 128, nbH = a.H / 128;
    a.nblk_h = a.H / 128;
    a.nblk_i = a.I / 128;
    a.P_gu = moe_splits(max_items < 16 ? max_items * nbI : 16 * nbI, a.nblk_h);
    a.P_d = moe_splits(max_items < 16 ? max_items * nbH : 16 * nbH, a.nblk_i);
    const int MR = a.MR > 0 ? a.MR : 1;
    Workspace ws;
    const size_t n_gu = (size_t)max_items * nbI, n_d = (size_t)max_items * nbH;
    const bool use_mfma = a.max_blocks > 0;
    size_t bytes = carve_size(1, 4) + carve_size(max_items, sizeof(ItemDesc)) +
                   carve_size(a.max_blocks, sizeof(ItemDesc)) +
                   (use_mfma ? carve_size(npairs * 2 * a.H, 2) + carve_size(npairs * 2 * (a.H / 128), 4) +
                                   carve_size(npairs, 4) +
                                   carve_size(npairs * (a.I / 128), 4) + carve_size(3 * (size_t)a.max_blocks + 3, 4)
                             : 0) +
                   carve_size(npairs * 2, 4) + carve_size(npairs, 4) +
                   carve_size(a.M, 4) +
                   carve_size(npairs * a.I, 2) + carve_size(npairs * a.H, 4) +
                   carve_size(n_gu * a.P_gu * 2 * MR * 128, 4) + carve_size(n_d * a.P_d * MR * 128, 4);
    const size_t n_tok = (size_t)a.M * nbH;
    int rc = workspace(bytes, n_gu + n_d + n_tok, st, &ws);
    if (rc) return rc;
    Carve c{ws.scratch, ws.scratch_bytes};
    a.n_items = c.take<int>(1);
    ItemDesc* items = c.take<ItemDesc>(max_items);
    a.items = items;
    ItemDesc* blocks = a.max_blocks ? c.take<ItemDesc>(a.max_blocks) : nullptr;
    a.blocks = blocks;
    a.xh = use_mfma ? c.take<_Float16>(npairs * 2 * a.H) : nullptr;
    a.xsum = use_mfma ? c.take<float>(npairs * 2 * (a.H / 128)) : nullptr;
    a.asum = use_mfma ? c.take<float>(npairs * (a.I / 128)) : nullptr;
    a.pair_e = use_mfma ? c.take<int>(npairs) : nullptr;
    int* cls = use_mfma ? c.take<int>(3 * (size_t)a.max_blocks + 3) : nullptr;
    a.cls_list = cls;
    a.cls_cnt = cls ? cls + 3 * (size_t)a.max_blocks : nullptr;
    int* pb = c.take<int>(npairs * 2);
    a.pair_tok = pb;
    a.pair_of = pb + npairs;
    a.pair_w = c.take<float>(npairs);
    a.tok_nvalid = c.take<int>(a.M);
    a.abuf = c.take<uint16_t>(npairs * a.I);
    a.y = c.take<float>(npairs * a.H);
    a.part_gu = c.take<float>(n_gu * a.P_gu * 2 * MR * 128);
    a.part_d = c.take<float>(n_d * a.P_d * MR * 128);
    if (!a.part_d) return fail(EXL3_ERR_INVALID, "moe: workspace carve failed");
    a.cnt_gu = ws.counters;
    a.cnt_d = ws.counters + n_gu;
    a.cnt_tok = ws.counters + n_gu + n_d;

    RouteArgs r{};
    r.ids = a.ids;
    r.tw = a.tw;
    r.M = a.M;
    r.topk = a.topk;
    r.slots = a.slots;
    r.E = a.E;
    r.shared = a.shared;
    r.MR = a.MR;
    r.n_items = a.n_items;
    r.items = items;
    r.max_items = max_items;
    r.tables = a.tables;
    r.kmaps = a.kmaps;
    r.use_mfma = use_mfma;
    r.MB = kMfmaRows;
    r.blocks = blocks;
    r.max_blocks = a.max_blocks;
    r.cls_list = cls;
    r.cls_cnt = cls ? cls + 3 * (size_t)a.max_blocks : nullptr;
    r.pair_tok = a.pair_tok;
    r.pair_w = a.pair_w;
    r.pair_of = a.pair_of;
    r.pair_e = a.pair_e;
    r.tok_nvalid = a.tok_nvalid;
    r.out = a.out;
    r.out_ld = a.out_ld;
    r.out_f32 = a.out_f32;
    r.H = a.H;
    rc = launch_align(r, st);
    if (rc) return rc;
    if (use_mfma && (rc = launch_moe_mfma(a, st))) return rc;
    if (max_items > 0)
        EXL3_LAUNCH("moe_gateup", gateup_select(a.Kg, MR, a.planar), dim3(max_items * nbI, a.P_gu), dim3(256), 0, st,
                    a);
    if (max_items > 0)
        EXL3_LAUNCH("moe_down", down_select(a.Kd, MR, a.planar), dim3(max_items * nbH, a.P_d), dim3(256), 0, st, a);
    return EXL3_OK;
}

static int check_K(int K, const char* what) {
    if (K < 0 || K > 8) return fail(EXL3_ERR_UNSUPPORTED, "exl3_moe_forward: %s K=%d not in 0..8", what, K);
    return EXL3_OK;
}

}  // namespace exl3

namespace exl3 {

// ------------------------------------------------------------------------------------------------ expert blobs
// The reference's expert blob (glm/xpu/csrc/exl3_moe.n128.sycl:3-11, Geom at :56-68; packed by pack_expert,
// glm/xpu/exl3xpu/moe_offload.py:81-94): gate|up trellis words [H/16][2I/16][8K] (per tile-row the I/16 gate tiles,
// then the I/16 up tiles), down trellis [I/16][H/16][8K], then fp16 suh_g[H] suh_u[H] svh_g[I] svh_u[I] suh_d[I]
// svh_d[H]. Tables [9][E] (trellis, suh, svh per projection) from one blob address per expert.
__global__ void blob_tables_kernel(const int64_t* __restrict__ ptrs, int E, int64_t gu_bytes, int64_t d_bytes,
                                   int64_t H, int64_t I, int K, int64_t* __restrict__ tab) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int64_t b = ptrs[e], sg = b + gu_bytes + d_bytes;
    tab[0 * (int64_t)E + e] = b;                                   // gate trellis
    tab[1 * (int64_t)E + e] = sg;                                  // suh_g
    tab[2 * (int64_t)E + e] = sg + 4 * H;                          // svh_g
    tab[3 * (int64_t)E + e] = b + (I / 16) * 8 * K * 4;            // up trellis: I/16 tiles into every tile-row
    tab[4 * (int64_t)E + e] = sg + 2 * H;                          // suh_u
    tab[5 * (int64_t)E + e] = sg + 4 * H + 2 * I;                  // svh_u
    tab[6 * (int64_t)E + e] = b + gu_bytes;                        // down trellis
    tab[7 * (int64_t)E + e] = sg + 4 * H + 4 * I;                  // suh_d
    tab[8 * (int64_t)E + e] = sg + 4 * H + 6 * I;                  // svh_d
}

// In-place PLANAR4 -> tile order where they differ (D = K / gcd(K, 32) > 1: K = 3, 5, 6, 7; G = 8K / D periods of D
// words per tile): within every group of 4 consecutive tiles of a tile-row, word (tile t, period g, plane i) sits at
// 4G i + G t + g; in tile order it is word D g + i of tile t, at 8K t + D g + i (glm/xpu/exl3xpu/moe_offload.py:68-78,
// glm/xpu/pack_store.py:35-54). Workgroup per (expert, tile-row of gate|up then of down); the row's groups pass
// through LDS one at a time.
__global__ __launch_bounds__(256) void blob_unplanarize_kernel(const int64_t* __restrict__ ptrs, int64_t gu_bytes,
                                                               int H, int I, int K, int D) {
    __shared__ uint32_t g[4 * 8 * 8];
    const int e = blockIdx.x, row = blockIdx.y;
    const int rows_gu = H / 16;
    uint32_t* base = reinterpret_cast<uint32_t*>(ptrs[e]);
    int tiles;
    if (row < rows_gu) {
        tiles = 2 * I / 16;
        base += (size_t)row * tiles * 8 * K;
    } else {
        tiles = H / 16;
        base = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(base) + gu_bytes) + (size_t)(row - rows_gu) * tiles * 8 * K;
    }
    const int W = 32 * K, G = 8 * K / D;                          // words per group of 4 tiles, periods per tile
    for (int grp = 0; grp < tiles / 4; ++grp) {
        uint32_t* gp = base + (size_t)grp * W;
        for (int j = threadIdx.x; j < W; j += 256) g[j] = gp[j];
        __syncthreads();
        for (int n = threadIdx.x; n < W; n += 256) {                // natural word n = 8K t + D gg + i
            const int t = n / (8 * K), r = n - t * 8 * K, gg = r / D, i = r - gg * D;
            gp[n] = g[4 * G * i + G * t + gg];
        }
        __syncthreads();
    }
}

}  // namespace exl3

using namespace exl3;

// Argument checks and MoeArgs shared by the two layer entry points (ids / weights may still be unset).
static int moe_setup(const uint16_t* x, int64_t x_ld, int64_t M, int64_t H, int64_t I, int64_t topk, int64_t E,
                     const int64_t* tables, const int64_t* kmaps, int K_gate, int K_up, int K_down, int act,
                     float act_limit, int64_t shared, void* out, int64_t out_ld, int out_dtype, MoeArgs& a) {
    int rc;
    if ((rc = check_K(K_gate, "gate")) || (rc = check_K(K_up, "up")) || (rc = check_K(K_down, "down"))) return rc;
    if (K_gate != K_up)
        return fail(EXL3_ERR_UNSUPPORTED, "exl3_moe_forward: gate and up must share K (got %d, %d)", K_gate, K_up);
    EXL3_CHECK_ARG(act == EXL3_ACT_SILU || act == EXL3_ACT_GELU_TANH, "exl3_moe_forward: unknown activation %d", act);
    EXL3_CHECK_ARG(out_dtype == EXL3_F16 || out_dtype == EXL3_F32, "exl3_moe_forward: out must be fp16 or fp32");
    EXL3_CHECK_ARG(M >= 0 && topk >= 0 && topk <= 64 && E > 0 && E <= kMoeMaxExperts,
                   "exl3_moe_forward: M=%lld topk=%lld E=%lld out of range", (long long)M, (long long)topk,
                   (long long)E);
    EXL3_CHECK_ARG(H > 0 && I > 0 && H % 128 == 0 && I % 128 == 0, "exl3_moe_forward: H and I must be multiples of 128");
    EXL3_CHECK_ARG(H / 16 * (I / 16) * 64 < (1LL << 32), "exl3_moe_forward: projection of %lld x %lld exceeds 2^32 words",
                   (long long)H, (long long)I);
    EXL3_CHECK_ARG(x_ld >= H && out_ld >= H, "exl3_moe_forward: row strides must cover H");
    EXL3_CHECK_ARG(shared < E, "exl3_moe_forward: shared expert index %lld >= E", (long long)shared);
    EXL3_CHECK_ARG(M == 0 || (x && tables && out), "exl3_moe_forward: null pointer");
    EXL3_CHECK_ARG(K_gate != 0 && K_down != 0 ? true : kmaps != nullptr,
                   "exl3_moe_forward: per-tile K (K=0) needs the kmaps table");
    a = MoeArgs{};
    a.x = x;
    a.x_ld = x_ld;
    a.M = (int)M;
    a.H = (int)H;
    a.I = (int)I;
    a.topk = (int)topk;
    a.slots = (int)topk + (shared >= 0 ? 1 : 0);
    a.E = (int)E;
    a.tables = tables;
    a.kmaps = kmaps;
    a.Kg = K_gate;
    a.Kd = K_down;
    a.gu_tn = (int)(I / 16);
    a.act = act;
    a.limit = act_limit;
    a.shared = (int)shared;
    a.out = out;
    a.out_ld = out_ld;
    a.out_f32 = out_dtype == EXL3_F32;
    return EXL3_OK;
}

static int moe_run(MoeArgs& a, hipStream_t st) {
    if (moe_fused_take(a)) return moe_fused_path(a, st);
    // GEMV items of up to MR rows per expert for decode batches (M <= 8), sparse batches of any size (pairs <= E / 2:
    // an expert takes one or two rows) and, with uniform K, batches of up to 16 tokens, up to 32 when the experts
    // are small (H * I <= 2^22), and up to 128 when the MFMA grid would be thin (active experts * I / 128 < 160
    // gate|up workgroups: 8 experts top-2, 128 tokens 116 -> 74 us; 32 experts top-4, 96 tokens 101 -> 87). Other prefill batches: every expert with rows goes to the MFMA kernels in blocks of up to
    // kMfmaRows rows (MR = 0: no GEMV items). Measured against the MFMA path: 512 experts of 2048 -> 512, top-10,
    // 16 / 20 / 25 tokens 141.5 -> 100.6, 153.5 -> 118.8, 165.6 -> 141.6 us; 16 experts top-9, 16 tokens 90.9 ->
    // 56.0; 8 experts top-8, 32 tokens 117.6 -> 72.5; 129 experts of 4096 -> 1408 with a shared one, 16 tokens
    // 254.6 -> 223.6; one expert of 4096 -> 4096, 32 / 64 tokens 176 -> 77, 210 -> 125; 8 experts top-2, 64 tokens
    // 103 -> 50. The MFMA path stays ahead for wide experts taking several rows each (16 experts of 4096 -> 4096,
    // top-4, 32 tokens 202 against 262 us on items), for grids of a few hundred workgroups or more past 32 tokens
    // (64 experts top-8, 64 tokens: 99 against 115), past 128 tokens, and for per-tile K (256 experts of 7168 -> 2048
    // with a shared one, 16 tokens 729 against 1064). EXL3MI_MOE_MFMA=1 forces the MFMA path at any batch size.
    const int64_t M = a.M, E = a.E, npairs = M * a.slots;
    bool mfma = M > kMoeSmallRows && npairs * 2 > E;
    if (mfma && M <= 128 && a.Kg > 0 && a.Kd > 0) {
        const bool small = (int64_t)a.H * a.I <= ((int64_t)1 << 22);
        const bool thin = moe_expected_items(a, 64) * (a.I / 128) < 160.0;   // one MFMA block per active expert
        mfma = !(M <= 16 || (M <= 32 && small) || thin);
    }
    // Per-tile K over wide experts: the MFMA mix kernels' K 1 / 2 fast path outruns the GEMV items' per-tile decode
    // once enough experts are active to amortise a block's unsplit k loop (256 experts of 7168 -> 2048 with a shared
    // one: 8 / 10 tokens, about 62 / 75 active, 618 -> 491, 731 -> 557 us on MFMA; 2 / 4 tokens, 17 / 33 active, stay
    // on items: 218 / 358 against 295 / 398).
    if (!mfma && (a.Kg == 0 || a.Kd == 0) && (int64_t)a.H * a.I > ((int64_t)1 << 22) &&
        moe_expected_items(a, 64) >= 48.0)
        mfma = true;
    if (env_int("EXL3MI_MOE_MFMA", 0)) mfma = true;
    a.MR = mfma ? 0 : M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : kMoeSmallRows;
    // rows per GEMV item: one for sparse routing (pairs <= E / 2; experts of 2048 -> 512, 8 tokens, against eight rows
    // per item: 512 experts top-17 170.6 -> 86.6 us), two up to 1.5 pairs per expert (128 experts top-17 78.7 against
    // 83.2 with four, 86.0 with one), else four: eight never pays on this path, even with every expert taking all 8
    // rows (8 experts top-8 34.5 us with four, 43.9 with eight; 32 experts top-32 83.0 with four, 102.4 with two;
    // 64 experts top-17 69.9 with four, 72.8 with two, 105.7 with eight). EXL3MI_MOE_MR=1|2|4|8 overrides.
    if (!mfma) {
        int cap = npairs * 2 <= E ? 1 : npairs * 2 <= 3 * E ? 2 : 4;
        // wide experts (H * I > 2^22) under sparse routing: two rows per item when that saves 8 % of the expected
        // items (a shared expert's rows pair up): 256 experts of 7168 -> 2048 (per-tile K) with a shared one, 4 / 8
        // tokens 377 -> 358.7, 686 -> 618 us; 160 experts of 5120 -> 1536, 8 tokens 182 -> 170.6; 129 experts of
        // 4096 -> 1408 with a shared one, 4 tokens 94.2 -> 91.3 (2 tokens of the first, 7 % fewer items: 218 at one
        // row, 221 at two)
        if (cap == 1 && M >= 2 && (int64_t)a.H * a.I > ((int64_t)1 << 22) &&
            moe_expected_items(a, 2) <= 0.92 * moe_expected_items(a, 1))
            cap = 2;
        // wide experts taking many rows each, past 16 tokens: eight rows per item while at least 8 items remain (one
        // expert of 4096 -> 4096, 64 / 128 tokens 124.5 -> 114, 220 -> 190 us; 4 experts top-2, 64 tokens 232 ->
        // 210.5; with 4 items left four rows win: one expert at 32 tokens 76 against 86)
        if (cap == 4 && M > 16 && (int64_t)a.H * a.I > ((int64_t)1 << 22) && moe_expected_items(a, 8) >= 8.0)
            cap = 8;
        if (a.MR > cap) a.MR = cap;
        const int mr_env = env_int("EXL3MI_MOE_MR", 0);
        if (mr_env == 1 || mr_env == 2 || mr_env == 4 || mr_env == 8) a.MR = mr_env;
    }
    int64_t mi = mfma ? 0 : E + npairs / a.MR;
    if (mi > npairs) mi = npairs;
    a.max_items = (int)mi;
    a.max_blocks = mfma ? (int)(npairs / kMfmaRows + (E < npairs ? E : npairs) + 1) : 0;
    EXL3_CHECK_ARG((int64_t)a.max_items * (a.H / 128) < 0x7FFFFFFF && a.max_blocks <= 65535,
                   "exl3_moe_forward: grid too large");
    return moe_decode_path(a, npairs, st);
}

extern "C" {

int exl3_moe_forward(const uint16_t* x, int64_t x_ld, int64_t M, int64_t H, int64_t I, const int32_t* topk_ids,
                     const float* topk_w, int64_t topk, int64_t E, const int64_t* tables, const int64_t* kmaps,
                     int K_gate, int K_up, int K_down, int act, float act_limit, int64_t shared, void* out,
                     int64_t out_ld, int out_dtype, void* stream) {
    MoeArgs a;
    int rc = moe_setup(x, x_ld, M, H, I, topk, E, tables, kmaps, K_gate, K_up, K_down, act, act_limit, shared, out,
                       out_ld, out_dtype, a);
    if (rc) return rc;
    if (M == 0) return EXL3_OK;
    EXL3_CHECK_ARG(topk == 0 || (topk_ids && topk_w), "exl3_moe_forward: null pointer");
    a.ids = topk_ids;
    a.tw = topk_w;
    return moe_run(a, (hipStream_t)stream);
}

// D = K / gcd(K, 32): words per period of the PLANAR4 order (1: the order is tile order)
static int planar_d(int K) { return K / (K & -K); }

int exl3_moe_forward_blobs(const uint16_t* x, int64_t x_ld, int64_t M, int64_t H, int64_t I, const int32_t* topk_ids,
                           const float* topk_w, int64_t topk, int64_t E, const int64_t* ptrs, int K, int act,
                           float act_limit, void* out, int64_t out_ld, int out_dtype, int word_order, void* stream) {
    if (K < 1 || K > 8) return fail(EXL3_ERR_UNSUPPORTED, "exl3_moe_forward_blobs: K=%d not in 1..8", K);
    EXL3_CHECK_ARG(word_order == EXL3_WORDS_PLANAR4 || word_order == EXL3_WORDS_TILE_ORDER,
                   "exl3_moe_forward_blobs: unknown word order %d", word_order);
    EXL3_CHECK_ARG(E > 0 && E <= kMoeMaxExperts && H > 0 && I > 0 && H % 128 == 0 && I % 128 == 0,
                   "exl3_moe_forward_blobs: E=%lld, H=%lld, I=%lld out of range", (long long)E, (long long)H,
                   (long long)I);
    EXL3_CHECK_ARG(H / 16 * (2 * I / 16) * 8 * K < (1LL << 32), "exl3_moe_forward_blobs: blob trellis exceeds 2^32 words");
    if (M == 0) return EXL3_OK;
    EXL3_CHECK_ARG(ptrs && topk_ids && topk_w, "exl3_moe_forward_blobs: null pointer");
    hipStream_t st = (hipStream_t)stream;
    void* tb = nullptr;
    int rc = aux_buffer((size_t)9 * E * sizeof(int64_t), st, &tb);
    if (rc) return rc;
    int64_t* tables = reinterpret_cast<int64_t*>(tb);
    const int64_t gu_bytes = H / 16 * (2 * I / 16) * 8 * K * 4, d_bytes = I / 16 * (H / 16) * 8 * K * 4;
    EXL3_LAUNCH("blob_tables", blob_tables_kernel, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, st, ptrs, (int)E,
                gu_bytes, d_bytes, H, I, K, tables);
    MoeArgs a;
    rc = moe_setup(x, x_ld, M, H, I, topk, E, tables, nullptr, K, K, K, act, act_limit, -1, out, out_ld, out_dtype, a);
    if (rc) return rc;
    a.gu_tn = (int)(2 * I / 16);
    a.planar = word_order == EXL3_WORDS_PLANAR4 && planar_d(K) > 1;
    a.ids = topk_ids;
    a.tw = topk_w;
    return moe_run(a, st);
}

int exl3_blob_unplanarize(const int64_t* ptrs, int64_t E, int64_t H, int64_t I, int K, void* stream) {
    if (K < 1 || K > 8) return fail(EXL3_ERR_UNSUPPORTED, "exl3_blob_unplanarize: K=%d not in 1..8", K);
    EXL3_CHECK_ARG(E > 0 && E <= 65535 && H > 0 && I > 0 && H % 128 == 0 && I % 128 == 0 && H / 16 + I / 16 <= 65535,
                   "exl3_blob_unplanarize: E=%lld, H=%lld, I=%lld out of range", (long long)E, (long long)H,
                   (long long)I);
    if (planar_d(K) == 1) return EXL3_OK;                          // K = 1, 2, 4, 8: already in tile order
    EXL3_CHECK_ARG(ptrs, "exl3_blob_unplanarize: null pointer");
    const int64_t gu_bytes = H / 16 * (2 * I / 16) * 8 * K * 4;
    EXL3_LAUNCH("blob_unplanarize", blob_unplanarize_kernel, dim3((unsigned)E, (unsigned)(H / 16 + I / 16)), dim3(256),
                0, (hipStream_t)stream, ptrs, gu_bytes, (int)H, (int)I, K, planar_d(K));
    return EXL3_OK;
}

int exl3_moe_forward_logits(const uint16_t* x, int64_t x_ld, int64_t M, int64_t H, int64_t I, const float* logits,
                            int64_t logits_ld, int64_t n_logits, const float* bias, int64_t topk, int64_t E,
                            const int64_t* tables, const int64_t* kmaps, int K_gate, int K_up, int K_down, int act,
                            float act_limit, int64_t shared, const int64_t* table_layout, int32_t* ids_out,
                            float* w_out, void* out, int64_t out_ld, int out_dtype, void* stream) {
    MoeArgs a;
    int rc = moe_setup(x, x_ld, M, H, I, topk, E, tables, kmaps, K_gate, K_up, K_down, act, act_limit, shared, out,
                       out_ld, out_dtype, a);
    if (rc) return rc;
    EXL3_CHECK_ARG(topk > 0 && topk <= 32 && n_logits >= topk && n_logits <= E && n_logits <= 8192 &&
                   logits_ld >= n_logits, "exl3_moe_forward_logits: bad router sizes (topk %lld, %lld logits, E %lld)",
                   (long long)topk, (long long)n_logits, (long long)E);
    if (M == 0) return EXL3_OK;
    EXL3_CHECK_ARG(logits && ids_out && w_out, "exl3_moe_forward_logits: null pointer");
    a.ids = ids_out;
    a.tw = w_out;
    if (table_layout) {
        a.uniform = 1;
        for (int i = 0; i < 9; ++i) {
            a.tb[i] = table_layout[i];
            a.ts[i] = table_layout[9 + i];
        }
    }
    // Batches of up to kFusedRouteMaxRows tokens on the fused layer rank the logits inside it: every workgroup ranks
    // the tokens itself (with one row per item just those of its own two items), which costs less than the router
    // launch (512 experts, top-10: 1 token 24.1 us against 25.0 with two-row items; with one-row items 3 tokens 28.4
    // against 30.2, 4 tokens 32.0 against 33.7) until the rankings in every workgroup outweigh it (8 tokens: 47.4
    // against 46.2). Otherwise the router kernel runs first.
    if (M <= kFusedRouteMaxRows && moe_fused_take(a) && n_logits <= kFusedRouteMaxE &&
        env_int("EXL3MI_ROUTER_KERNEL", 0) == 0) {
        a.logits = logits;
        a.lg_ld = logits_ld;
        a.n_logits = (int)n_logits;
        a.rbias = bias;
        a.ids_out = ids_out;
        a.tw_out = w_out;
        return moe_run(a, (hipStream_t)stream);
    }
    if ((rc = exl3_route_softmax_topk(logits, logits_ld, M, n_logits, bias, topk, ids_out, w_out, stream))) return rc;
    return moe_run(a, (hipStream_t)stream);
}

int exl3_moe_align(const int32_t* topk_ids, const float* topk_w, int64_t M, int64_t topk, int64_t E, int64_t shared,
                   int32_t* counts, int32_t* pair_tok, float* pair_w, int32_t* pair_of, void* stream) {
    EXL3_CHECK_ARG(M >= 0 && topk >= 0 && E > 0 && E <= kMoeMaxExperts && shared < E, "exl3_moe_align: bad sizes");
    if (M == 0) return EXL3_OK;
    EXL3_CHECK_ARG(topk_ids && topk_w && counts && pair_tok && pair_w && pair_of, "exl3_moe_align: null pointer");
    RouteArgs r{};
    r.ids = topk_ids;
    r.tw = topk_w;
    r.M = (int)M;
    r.topk = (int)topk;
    r.slots = (int)topk + (shared >= 0 ? 1 : 0);
    r.E = (int)E;
    r.shared = (int)shared;
    r.MR = 1;
    r.counts = counts;
    r.pair_tok = pair_tok;
    r.pair_w = pair_w;
    r.pair_of = pair_of;
    return launch_align(r, (hipStream_t)stream);
}

int exl3_act_mul(const void* x, const void* y, uint16_t* z, int64_t n, int dtype, int act, float act_limit,
                 void* stream) {
    EXL3_CHECK_ARG(dtype == EXL3_F16 || dtype == EXL3_F32, "exl3_act_mul: dtype must be fp16 or fp32");
    EXL3_CHECK_ARG(act == EXL3_ACT_SILU || act == EXL3_ACT_GELU_TANH, "exl3_act_mul: unknown activation %d", act);
    EXL3_CHECK_ARG(n >= 0, "exl3_act_mul: negative size");
    if (n == 0) return EXL3_OK;
    EXL3_CHECK_ARG(x && y && z, "exl3_act_mul: null pointer");
    const int64_t blocks = (n + 255) / 256;
    EXL3_CHECK_ARG(blocks <= 0x7FFFFFFF, "exl3_act_mul: too large");
    if (dtype == EXL3_F16)
        EXL3_LAUNCH("act_mul", act_mul_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, x, y,
                    z, n, act, act_limit);
    else
        EXL3_LAUNCH("act_mul", act_mul_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, x, y,
                    z, n, act, act_limit);
    return EXL3_OK;
}

int exl3_route_topk(const float* logits, int64_t ld, int64_t M, int64_t E, const float* bias, int64_t k, int score,
                    int flags, float scaling, int32_t* ids, float* w, void* stream) {
    EXL3_CHECK_ARG(M >= 0 && E > 0 && E <= 8192 && k > 0 && k <= 32 && k <= E && ld >= E,
                   "exl3_route_topk: bad sizes (M %lld, E %lld, k %lld, ld %lld)", (long long)M, (long long)E,
                   (long long)k, (long long)ld);
    if (score != EXL3_SCORE_SOFTMAX && score != EXL3_SCORE_SIGMOID && score != EXL3_SCORE_SQRT_SOFTPLUS)
        return fail(EXL3_ERR_UNSUPPORTED, "exl3_route_topk: scoring %d not supported", score);
    EXL3_CHECK_ARG((flags & ~(EXL3_ROUTE_RENORM | EXL3_ROUTE_BIAS_SELECT_ONLY)) == 0, "exl3_route_topk: bad flags %d",
                   flags);
    if (M == 0) return EXL3_OK;
    EXL3_CHECK_ARG(logits && ids && w, "exl3_route_topk: null pointer");
    EXL3_CHECK_ARG(M <= 0x7FFFFFFF, "exl3_route_topk: too many rows");
    route_fn kern = score == EXL3_SCORE_SOFTMAX ? route_pick<EXL3_SCORE_SOFTMAX>(E)
                  : score == EXL3_SCORE_SIGMOID ? route_pick<EXL3_SCORE_SIGMOID>(E)
                  : route_pick<EXL3_SCORE_SQRT_SOFTPLUS>(E);
    EXL3_LAUNCH("route_topk", kern, dim3((unsigned)M), dim3(64), 0, (hipStream_t)stream, logits, ld, (int)E, bias,
                (int)k, flags, scaling, ids, w);
    return EXL3_OK;
}

int exl3_route_adjusted(const float* logits, int64_t ld, int64_t M, int64_t E, const float* bias, const float* mul,
                        const float* res, int64_t k, int score, int flags, float scaling, int32_t* ids, float* w,
                        void* stream) {
    EXL3_CHECK_ARG(M >= 0 && E > 0 && E <= 2048 && k > 0 && k <= 32 && k <= E && ld >= E,
                   "exl3_route_adjusted: bad sizes (M %lld, E %lld, k %lld, ld %lld)", (long long)M, (long long)E,
                   (long long)k, (long long)ld);
    if (score != EXL3_SCORE_SIGMOID && score != EXL3_SCORE_SQRT_SOFTPLUS)
        return fail(EXL3_ERR_UNSUPPORTED, "exl3_route_adjusted: scoring %d (sigmoid or sqrt-softplus only)", score);
    EXL3_CHECK_ARG((flags & ~EXL3_ROUTE_RENORM) == 0, "exl3_route_adjusted: bad flags %d", flags);
    if (M == 0) return EXL3_OK;
    EXL3_CHECK_ARG(logits && ids && w, "exl3_route_adjusted: null pointer");
    EXL3_CHECK_ARG(M <= 0x7FFFFFFF, "exl3_route_adjusted: too many rows");
    route_adj_fn kern = score == EXL3_SCORE_SIGMOID ? route_adj_pick<EXL3_SCORE_SIGMOID>(E)
                                                    : route_adj_pick<EXL3_SCORE_SQRT_SOFTPLUS>(E);
    EXL3_LAUNCH("route_adjusted", kern, dim3((unsigned)M), dim3(64), 0, (hipStream_t)stream, logits, ld, (int)E, bias,
                mul, res, (int)k, flags, scaling, ids, w);
    return EXL3_OK;
}

int exl3_route_block(const float* logits, int64_t ld, int64_t M, int64_t E, const float* bias, const float* mul,
                     int64_t k, int64_t rows_per_block, float block_boost, float scaling, int32_t* ids, float* w,
                     void* stream) {
    EXL3_CHECK_ARG(M >= 0 && E > 0 && E <= 2048 && k > 0 && k <= 32 && k <= E && ld >= E,
                   "exl3_route_block: bad sizes (M %lld, E %lld, k %lld, ld %lld)", (long long)M, (long long)E,
                   (long long)k, (long long)ld);
    EXL3_CHECK_ARG(rows_per_block >= 1 && M % rows_per_block == 0 && rows_per_block <= 65536,
                   "exl3_route_block: %lld rows do not split into blocks of %lld", (long long)M,
                   (long long)rows_per_block);
    if (M == 0) return EXL3_OK;
    EXL3_CHECK_ARG(logits && ids && w, "exl3_route_block: null pointer");
    EXL3_CHECK_ARG(M / rows_per_block <= 0x7FFFFFFF, "exl3_route_block: too many blocks");
    route_block_fn kern = E <= 64 ? route_block_kernel<1> : E <= 128 ? route_block_kernel<2>
                        : E <= 256 ? route_block_kernel<4> : E <= 512 ? route_block_kernel<8>
                        : E <= 1024 ? route_block_kernel<16> : route_block_kernel<32>;
    EXL3_LAUNCH("route_block", kern, dim3((unsigned)(M / rows_per_block)), dim3(64), 0, (hipStream_t)stream, logits,
                ld, (int)E, bias, mul, (int)k, (int)rows_per_block, block_boost, scaling, ids, w);
    return EXL3_OK;
}

int exl3_route_softmax_topk(const float* logits, int64_t ld, int64_t M, int64_t E, const float* bias, int64_t k,
                            int32_t* ids, float* w, void* stream) {
    return exl3_route_topk(logits, ld, M, E, bias, k, EXL3_SCORE_SOFTMAX, EXL3_ROUTE_RENORM, 1.0f, ids, w, stream);
}

int exl3_router_logits(const uint16_t* x, int64_t x_ld, int64_t M, int64_t H, const uint16_t* W, int64_t w_ld,
                       int64_t E, int w_layout, int round_fp16, float* logits, int64_t logits_ld, void* stream) {
    EXL3_CHECK_ARG(M >= 0 && H > 0 && H % 128 == 0 && E > 0 && E <= 65536 && x_ld >= H && logits_ld >= E,
                   "exl3_router_logits: bad sizes (M %lld, H %lld, E %lld)", (long long)M, (long long)H, (long long)E);
    EXL3_CHECK_ARG(w_layout == EXL3_ROUTER_W_HE || w_layout == EXL3_ROUTER_W_EH, "exl3_router_logits: bad w_layout %d",
                   w_layout);
    if (M == 0) return EXL3_OK;
    EXL3_CHECK_ARG(x && W && logits, "exl3_router_logits: null pointer");
    EXL3_CHECK_ARG(M <= 4 * 65535 && H <= 0x7FFFFFFF, "exl3_router_logits: shape too large");
    EXL3_CHECK_ARG(aligned(W, 16) && w_ld % 8 == 0, "exl3_router_logits: W must be 16-byte aligned, row stride a multiple of 8");
    hipStream_t st = (hipStream_t)stream;
    const int MR = M >= 8 ? 8 : M >= 4 ? 4 : M >= 2 ? 2 : 1;       // rows per workgroup ([H, E]: at most 4)
    typedef void (*rfn)(const uint16_t*, int64_t, int, int, const uint16_t*, int64_t, int, int, float*, int64_t);
    if (w_layout == EXL3_ROUTER_W_HE) {
        EXL3_CHECK_ARG(E % 8 == 0 && w_ld >= E && aligned(x, 4) && x_ld % 2 == 0,
                       "exl3_router_logits: [H, E] weights need E a multiple of 8, w_ld >= E and a 4-byte aligned x");
        const int mr = MR > 4 ? 4 : MR;
        rfn fn = mr == 4 ? router_cols_kernel<4> : mr == 2 ? router_cols_kernel<2> : router_cols_kernel<1>;
        const unsigned gy = (unsigned)((M + mr - 1) / mr);
        EXL3_LAUNCH("router_logits", fn, dim3((unsigned)((E + 63) / 64), gy), dim3(1024), 0, st, x, x_ld, (int)M,
                    (int)H, W, w_ld, (int)E, round_fp16 ? 1 : 0, logits, logits_ld);
    } else {
        EXL3_CHECK_ARG(w_ld >= H && aligned(x, 16) && x_ld % 8 == 0,
                       "exl3_router_logits: [E, H] weights need w_ld >= H and a 16-byte aligned x (row stride a multiple of 8)");
        rfn fn = MR == 8 ? router_rows_kernel<8> : MR == 4 ? router_rows_kernel<4> : MR == 2 ? router_rows_kernel<2>
                                                                                          : router_rows_kernel<1>;
        const unsigned gy = (unsigned)((M + MR - 1) / MR);
        EXL3_LAUNCH("router_logits", fn, dim3((unsigned)((E + 3) / 4), gy), dim3(256), 0, st, x, x_ld, (int)M, (int)H,
                    W, w_ld, (int)E, round_fp16 ? 1 : 0, logits, logits_ld);
    }
    return EXL3_OK;
}

}  // extern "C"
