// Fused small-batch MoE layer on gfx950: gate|up, activation, down and combine in ONE launch.
//
// For decode batches (at most 16 tokens, at most kFusedMaxPairs (token, slot) pairs) the multi-kernel path is a chain
// of short latency-bound launches. Here every workgroup:
//   1. reads the routing ids (or, given router logits, ranks them itself: every wave one token, the picks in LDS) and
//      groups the pairs (pair l in lanes l and l + 64 of wave 0) by expert in
//      registers, once: a pair's index among its expert's pairs in flat order comes from an LDS sweep, items are
//      chunks of up to MR such pairs (the reference's per-expert row groups, glm/xpu/csrc/exl3_moe.n128.sycl:691-734)
//      numbered by a ballot over their first pairs, and an item's expert and rows follow from ballots. No align
//      launch; rows keep their flat pair index as row id.
//   2. runs gate|up job blockIdx.x (item i = blockIdx.x / GU; GU jobs per item = 128-column blocks of I x k-splits of
//      H in tile-rows), then the down jobs of item i - 1 (DN per item = 128-column blocks of H x k-splits of I; job
//      r of that item on the workgroup with r = blockIdx.x - i GU (mod GU)). A gate|up job streams both strips and,
//      in the last split to arrive, applies the reference's GateUpKernel epilogue (Hadamard * svh, act, * suh_d,
//      Hadamard: exl3_moe.n128.sycl:253-271) and publishes the item's down input. A down job prefetches its first
//      weight rows, waits until every column block of its item's down input is published, streams, and writes the
//      weighted rows y (directly when I is not split, else in the last split); the workgroup that completes a token's
//      slots sums them in slot order (exl3_moe.n128.sycl:385-410).
// Progress: gate|up jobs never wait, and a down job of item i only waits for the gate|up jobs of item i, which run on
// workgroups with lower ids ([i GU, (i + 1) GU) against >= (i + 1) GU). Workgroups are dispatched in id order within
// each XCD (ids round-robin over the XCDs), and every workgroup finishes its gate|up job before it can wait, so the
// lowest waiting workgroup always has its inputs coming: no co-residency is assumed. The grid is sized to what the
// device holds at once, so in practice every workgroup is resident from the start. The wait is also bounded: a
// timeout sets the device's host-mapped status word instead of hanging (the job then runs on incomplete inputs and
// the counters may be left non-zero; the next library call on the device finds the word on the host, zeroes the
// counters and fails with EXL3_ERR_HIP). Cross-workgroup data (partials, down inputs, y) moves with
// agent-scope stores and loads that write through the XCD-local L2, published by counters after the stores have
// drained (the split-K handoff). Every counter sits on its own 128-byte line.
#pragma once

#include "exl3_device.h"
#include "exl3_gemv.h"
#include "exl3_moe.h"
#include "exl3_moe_dev.h"
#include "exl3_runtime.h"

namespace exl3 {

constexpr int kFusedMaxPairs = 128;
constexpr int kFusedMaxRows = 16;     // tokens (items still hold at most 8 rows)
constexpr int kFusedMinJobRows = 20;    // tile-rows of H per gate|up job, at least
constexpr int kCS = 32;                 // counter stride in ints (one 128-byte line per counter)
#ifndef EXL3_FUSED_RING
#define EXL3_FUSED_RING 4
#endif
constexpr int kFusedRing = EXL3_FUSED_RING;   // GEMV register ring depth (loads run kFusedRing - 1 tile-rows ahead)

struct FusedArgs {
    const uint16_t* x;
    int64_t x_ld;
    int M, H, I, topk, slots, E, shared, np;
    const int32_t* ids;
    const float* tw;
    const int64_t* tables;              // [9][E]
    const int64_t* kmaps;               // [6][E] or null
    int act;
    float limit;
    float* abuf;                        // [max_items][MR][I] down input (fp16 values held in fp32)
    float* y;                           // [np][H] weighted expert outputs
    float* part_gu;                     // [max_items * nbI][P_gu][2][MR][128]
    float* part_d;                      // [max_items * nbH][P_d][MR][128] (P_d > 1)
    int* cnt_gu;                        // [max_items * nbI] * kCS
    int* cnt_d;                         // [max_items * nbH] * kCS
    int* cnt_tok;                       // [M * nbH] * kCS
    int* cnt_item;                      // [max_items] * kCS
    int* status;                        // host-mapped status word, set when a wait gives up (report_timeout)
    int spin_max;                       // polls of a down job's wait before it gives up (each backs off <= ~512 cycles)
    int P_gu, P_d;                      // k-splits (in tile-rows) of H for gate|up and of I for down
    int direct;                         // down jobs build their inputs from the gate|up partials (no epilogue stage)
    int uniform;                        // expert e's table entry i is tb[i] + e * ts[i] (no table loads)
    int64_t tb[9], ts[9];
    int GU, DN;                         // gate|up jobs (I / 128 * P_gu) and down jobs (H / 128 * P_d) per item
    int gu_tn;                          // tiles per tile-row of the gate and up trellises (MoeArgs::gu_tn)
    int J_gu, max_items;
    void* out;
    int64_t out_ld;
    int out_f32;
    // in-layer routing (logits non-null): every workgroup ranks the logits itself (the picks stay in LDS) and
    // workgroup 0 writes them to ids_out / tw_out
    const float* logits;
    int64_t lg_ld;
    int n_logits;
    const float* rbias;
    int32_t* ids_out;
    float* tw_out;
};

__device__ __forceinline__ int atomic_add_agent(int* p, int v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int atomic_load_agent(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_store_agent(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int MR>
struct FusedShared {
    static constexpr int KBF = MR <= 4 ? 8 : 4;        // 128-blocks of x a job stages (its k range, block-aligned)
    _Float16 xs[2][MR][KBF * 128];
    float red[4][MR][2][64];
    float cv[MR][128];                  // down outputs of an unsplit down job, natural column order
    float ksum[2][MR];                  // per projection and row: sum of the transformed x over the job's k range
    _Float16 su[2][KBF * 128];          // gate / up input sign vectors of the staged blocks
    int ge[kFusedMaxPairs];             // the pairs' experts (grouping sweep of wave 0)
    int rid[kFusedMaxPairs];            // in-layer routing: expert of pick (token, j) at token * topk + j
    float rw[kFusedMaxPairs];           //   and its weight
    int64_t tab[9];                     // the item's (trellis, suh, svh) addresses for gate, up, down
    int64_t km[6];                      // the item's (kmap, woff) addresses when K is per tile
    uint64_t valid[2];                  // valid pairs
    int rows[MR];                       // flat pair index of each row of the job's item
    int comb[MR];
    int nitems, it_e, it_cnt;
    int flag;
};

// k range of split p of P over T tile-rows, and the 128-blocks that cover it
struct KRange {
    int t0, nt;                         // first tile-row, tile-rows
    int b0, kbs;                        // first staged block, staged blocks
    int xo;                             // offset of tile-row t0 in the staged blocks (elements)
};
__device__ __forceinline__ KRange k_range(int p, int P, int T) {
    KRange r;
    r.t0 = (int)((int64_t)p * T / P);
    const int t1 = (int)((int64_t)(p + 1) * T / P);
    r.nt = t1 - r.t0;
    r.b0 = r.t0 >> 3;
    r.kbs = ((t1 + 7) >> 3) - r.b0;
    r.xo = 16 * r.t0 - 128 * r.b0;
    return r;
}

// The pair grouping as the grouping wave holds it (per-lane values for pairs lane and lane + 64, uniform masks).
struct Groups {
    int e0, e1, bf0, bf1;               // expert and index among its expert's pairs of pairs lane, lane + 64
    uint64_t L0, L1;                    // pairs that start an item
    uint64_t v0, v1;                    // valid pairs
    int n0, nitems;
};

// The job's item as every wave reads it from LDS (uniform values; its rows are in FusedShared::rows).
struct Item {
    int e, cnt;                         // expert, rows
    int64_t km[6];                      // (kmap, woff) addresses when K is per tile
};

// Expert of pair p, -1 for none (p >= np, a negative id, the absent shared expert). The id load is unconditional
// (clamped index) so that both of a lane's loads are in flight together.
// With in-layer routing the picks come from LDS (rid / rw), else from the ids / tw arrays.
__device__ __forceinline__ int pair_expert(const FusedArgs& a, int p, const int* rid) {
    const int pc = p < a.np ? p : a.np - 1;
    const int tok = pc / a.slots, j = pc - tok * a.slots;
    const int q = tok * a.topk + (j < a.topk ? j : a.topk - 1);
    const int v = a.topk <= 0 ? 0 : a.logits ? rid[q] : ldg(a.ids + q);
    const int e = j < a.topk ? v : a.shared;
    return p < a.np && e < a.E ? e : -1;
}

__device__ __forceinline__ float pair_weight(const FusedArgs& a, int p, const float* rw) {
    const int tok = p / a.slots, j = p - tok * a.slots;
    const int q = tok * a.topk + j;
    return j < a.topk ? (a.logits ? rw[q] : ldg(a.tw + q)) : 1.0f;
}

// In-layer routing of token t by one wave (softmax over logits + bias, top-k, renormalised: exl3_route_softmax_topk's
// route_row) into rid / rw; `out`: also write the picks out.
__device__ __forceinline__ void route_token(const FusedArgs& a, int t, int lane, int* rid, float* rw, bool out) {
    int id;
    float w;
    route_row<kFusedRouteMaxE / 64, EXL3_SCORE_SOFTMAX>(a.logits + (int64_t)t * a.lg_ld, a.rbias, a.n_logits, a.topk,
                                                       lane, true, true, 1.0f, id, w);
    if (lane < a.topk) {
        rid[t * a.topk + lane] = id;
        rw[t * a.topk + lane] = w;
        if (out) {
            a.ids_out[t * a.topk + lane] = id;
            a.tw_out[t * a.topk + lane] = w;
        }
    }
}

// Every token: wave w ranks tokens w, w + 4, ..; workgroup 0 writes the picks out.
__device__ __forceinline__ void route_in_layer(const FusedArgs& a, int wave, int lane, int* rid, float* rw) {
    for (int t = wave; t < a.M; t += 4) route_token(a, t, lane, rid, rw, blockIdx.x == 0);
}

__device__ __forceinline__ int popc64(uint64_t m) { return __popcll(m); }

__device__ __forceinline__ int ctz64(uint64_t m) { return __ffsll((unsigned long long)m) - 1; }
// set bits of (lo, hi) in [b, b + n) (a 128-bit mask; n <= 64)
__device__ __forceinline__ int popc_range(uint64_t lo, uint64_t hi, int b, int n) {
    int c = 0;
    for (int i = b; i < b + n; ++i) c += (int)(((i < 64 ? lo >> i : hi >> (i - 64))) & 1);
    return c;
}

// Groups the pairs (one wave; `ge` is a 128-int LDS array written and read by this wave only: LDS keeps a wave's
// accesses in order).
template <int MR>
__device__ __forceinline__ void group_pairs(const FusedArgs& a, int lane, Groups& g, int* ge, const int* rid) {
    const int l1 = lane + 64;
    g.e0 = pair_expert(a, lane, rid);
    g.e1 = pair_expert(a, l1, rid);
    int bf0 = 0, bf1 = 0;
    // one row per item: every valid pair starts an item, so no pair needs its index among its expert's pairs
    if constexpr (MR > 1) {
        ge[lane] = g.e0;
        ge[l1] = g.e1;
        for (int q4 = 0; q4 < a.np; q4 += 4) {        // entries past np are -1 and only match lanes without a pair
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ge + q4);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int eq = (int)v[k], q = q4 + k;
                bf0 += (eq == g.e0) & (q < lane);
                bf1 += (eq == g.e1) & (q < l1);
            }
        }
    }
    g.bf0 = bf0;
    g.bf1 = bf1;
    g.L0 = __ballot(g.e0 >= 0 && bf0 % MR == 0);
    g.L1 = __ballot(g.e1 >= 0 && bf1 % MR == 0);
    g.v0 = __ballot(g.e0 >= 0);
    g.v1 = __ballot(g.e1 >= 0);
    g.n0 = popc64(g.L0);
    g.nitems = g.n0 + popc64(g.L1);
}

// The (trellis, suh, svh) addresses of expert e for gate, up and down (and its kmaps when K is per tile) into LDS.
template <int K, int MR>
__device__ __forceinline__ void item_tables(const FusedArgs& a, int e, int lane, FusedShared<MR>& s) {
    if (lane < 9) {
        // uniform expert layout: entry i of expert e is at tb[i] + e * ts[i], no table load
        int64_t b = 0, st = 0;
#pragma unroll
        for (int i = 0; i < 9; ++i)
            if (lane == i) {
                b = a.tb[i];
                st = a.ts[i];
            }
        s.tab[lane] = a.uniform ? b + (int64_t)e * st : ldg(a.tables + (int64_t)lane * a.E + e);
    }
    if (K == 0 && lane < 6) s.km[lane] = ldg(a.kmaps + (int64_t)lane * a.E + e);
}

// One row per item with the routing ranked inside the layer: every pair is valid (the picks are experts < E and the
// shared slot, if any, names a valid expert) and starts an item, so item i is pair i and no grouping is needed. Every
// wave writes the item's description itself (the same values), so no barrier is needed before it reads them back:
// a wave's LDS accesses complete in order.
template <int K>
__device__ __forceinline__ void pair_item(const FusedArgs& a, int p, int lane, FusedShared<1>& s) {
    const int e = pair_expert(a, p, s.rid);
    if (lane == 0) {
        s.it_e = e;
        s.it_cnt = 1;
        s.rows[0] = p;
    }
    item_tables<K, 1>(a, e, lane, s);
}

// Expert, row count, rows, tables (and kmaps) of item `item` (< nitems) into LDS, by the wave that grouped the pairs;
// the other waves read them after a barrier (read_item).
template <int K, int MR>
__device__ __forceinline__ void item_info(const FusedArgs& a, const Groups& g, int item, int lane,
                                          FusedShared<MR>& s) {
    // first pair of the item: the item-th set bit of (L0, L1)
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    const uint64_t s0 = __ballot(((g.L0 >> lane) & 1) && popc64(g.L0 & below) == item);
    const uint64_t s1 = __ballot(((g.L1 >> lane) & 1) && g.n0 + popc64(g.L1 & below) == item);
    const int p = s0 ? ctz64(s0) : 64 + ctz64(s1);
    const int e = p < 64 ? __builtin_amdgcn_readlane(g.e0, p) : __builtin_amdgcn_readlane(g.e1, p - 64);
    const int bfp = p < 64 ? __builtin_amdgcn_readlane(g.bf0, p) : __builtin_amdgcn_readlane(g.bf1, p - 64);
    const int cnt = MR == 1 ? 1 : min(MR, popc64(__ballot(g.e0 == e)) + popc64(__ballot(g.e1 == e)) - bfp);
    if (lane == 0) {
        s.it_e = e;
        s.it_cnt = cnt;
    }
    item_tables<K, MR>(a, e, lane, s);
    if constexpr (MR == 1) {
        if (lane == 0) s.rows[0] = p;                    // the item is its first pair
    } else {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const uint64_t r0 = __ballot(g.e0 == e && g.bf0 == bfp + m), r1 = __ballot(g.e1 == e && g.bf1 == bfp + m);
            if (lane == 0) s.rows[m] = m < cnt ? (r0 ? ctz64(r0) : 64 + ctz64(r1)) : 0;
        }
    }
}

template <int K, int MR>
__device__ __forceinline__ Item read_item(const FusedShared<MR>& s) {
    Item it;
    it.e = s.it_e;
    it.cnt = s.it_cnt;
#pragma unroll
    for (int i = 0; i < 6; ++i) it.km[i] = K == 0 ? s.km[i] : 0;
    return it;
}

// sum over pp < P of the partials at base + pp * stride + off (agent-scope loads, issued 32 at a time, added in pp
// order)
template <int NV>
__device__ __forceinline__ void sum_partials(const float* base, size_t stride, const int (&off)[NV], int P,
                                             float (&acc)[NV]) {
    constexpr int B = 32 / NV;
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.f;
    for (int p0 = 0; p0 < P; p0 += B) {
        // unconditional loads (split index clamped to P - 1), so the whole batch is in flight before the first add
        float t[B][NV];
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int pp = p0 + i < P ? p0 + i : P - 1;
#pragma unroll
            for (int v = 0; v < NV; ++v) t[i][v] = splitk_load(base + (size_t)pp * stride + off[v]);
        }
#pragma unroll
        for (int i = 0; i < B; ++i)
#pragma unroll
            for (int v = 0; v < NV; ++v) acc[v] += p0 + i < P ? t[i][v] : 0.f;
    }
}

// The strip GEMV sized to the item's row count (wave-uniform): most decode items hold one row, and at 4 rows the dot
// products are a third of the GEMV's VALU work. Rows past the variant's size keep their zero accumulators.
template <int KL, int MR, bool PL = false>
__device__ __forceinline__ void item_gemv(int cnt, const uint32_t* sp, size_t rs, int lt0, int nt, int step, int lane,
                                          const _Float16* xs, int xs_ld, float (&acc)[MR][2],
                                          StripRing<KL, kFusedRing>& ring) {
    cnt = __builtin_amdgcn_readfirstlane(cnt);
    if constexpr (MR >= 2)
        if (cnt == 1) {
            strip_gemv_run<KL, 1, kFusedRing, PL>(sp, rs, lt0, nt, step, lane, xs, xs_ld,
                                              reinterpret_cast<float(&)[1][2]>(acc), ring);
            return;
        }
    if constexpr (MR >= 4)
        if (cnt == 2) {
            strip_gemv_run<KL, 2, kFusedRing, PL>(sp, rs, lt0, nt, step, lane, xs, xs_ld,
                                              reinterpret_cast<float(&)[2][2]>(acc), ring);
            return;
        }
    if constexpr (MR >= 8)
        if (cnt <= 4) {
            strip_gemv_run<KL, 4, kFusedRing, PL>(sp, rs, lt0, nt, step, lane, xs, xs_ld,
                                              reinterpret_cast<float(&)[4][2]>(acc), ring);
            return;
        }
    strip_gemv_run<KL, MR, kFusedRing, PL>(sp, rs, lt0, nt, step, lane, xs, xs_ld, acc, ring);
}

template <int MR>
__device__ __forceinline__ void item_gemv_mixed(int cnt, const uint32_t* words, const uint8_t* kmap,
                                                const int32_t* woff, int tn, int tile_n0, int tr0, int lt0, int nt,
                                                int step, int lane, const _Float16* xs, int xs_ld,
                                                float (&acc)[MR][2]) {
    cnt = __builtin_amdgcn_readfirstlane(cnt);
    if constexpr (MR >= 2)
        if (cnt == 1) {
            strip_gemv_mixed<1>(words, kmap, woff, tn, tile_n0, tr0, lt0, nt, step, lane, xs, xs_ld,
                                reinterpret_cast<float(&)[1][2]>(acc));
            return;
        }
    if constexpr (MR >= 4)
        if (cnt == 2) {
            strip_gemv_mixed<2>(words, kmap, woff, tn, tile_n0, tr0, lt0, nt, step, lane, xs, xs_ld,
                                reinterpret_cast<float(&)[2][2]>(acc));
            return;
        }
    if constexpr (MR >= 8)
        if (cnt <= 4) {
            strip_gemv_mixed<4>(words, kmap, woff, tn, tile_n0, tr0, lt0, nt, step, lane, xs, xs_ld,
                                reinterpret_cast<float(&)[4][2]>(acc));
            return;
        }
    strip_gemv_mixed<MR>(words, kmap, woff, tn, tile_n0, tr0, lt0, nt, step, lane, xs, xs_ld, acc);
}

// sum over the job's k range of the staged, transformed rows: ksum[proj][m] for the first `nproj` projections
template <int MR>
__device__ __forceinline__ void range_sums(FusedShared<MR>& s, int nproj, int cnt, const KRange& kr, int wave,
                                           int lane) {
    for (int i = wave; i < nproj * MR; i += 4) {
        const int pj = i / MR, m = i - pj * MR;
        float t = 0.f;
        if (m < cnt)
            for (int k = lane; k < 16 * kr.nt; k += 64) t += (float)s.xs[pj][m][kr.xo + k];
        t = wave_sum_f32(t);
        if (lane == 0) s.ksum[pj][m] = t;
    }
}

// Down input of row m, column block nb of I, from the gate|up partials of `slot` (the reference's GateUpKernel
// epilogue, exl3_moe.n128.sycl:253-271): sum of the P_gu partials in split order, Hadamard * svh for gate and up (fp16),
// act (fp16), * suh_d (fp16), Hadamard / sqrt(128) (fp16). Returns elements lane and lane + 64 (fp16 values in fp32).
template <int MR>
__device__ __forceinline__ void down_input(const FusedArgs& a, const int64_t* tab, size_t slot, int nb, int m, int lane,
                                           float& r0, float& r1) {
    const uint16_t* svg = reinterpret_cast<const uint16_t*>(tab[2]) + nb * 128;
    const uint16_t* svu = reinterpret_cast<const uint16_t*>(tab[5]) + nb * 128;
    const uint16_t* sud = reinterpret_cast<const uint16_t*>(tab[7]) + nb * 128;
    const float sg0 = h2f(ldg(svg + lane)), sg1 = h2f(ldg(svg + lane + 64));
    const float su0 = h2f(ldg(svu + lane)), su1 = h2f(ldg(svu + lane + 64));
    const float sd0 = h2f(ldg(sud + lane)), sd1 = h2f(ldg(sud + lane + 64));
    const int off[4] = {m * 128 + lane, m * 128 + lane + 64, (MR + m) * 128 + lane, (MR + m) * 128 + lane + 64};
    float v[4];
    sum_partials<4>(a.part_gu + slot * a.P_gu * 2 * MR * 128, 2 * MR * 128, off, a.P_gu, v);
    float g0 = v[0], g1 = v[1], u0 = v[2], u1 = v[3];
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
    r0 = (float)(_Float16)(a0 * kRsqrt128);
    r1 = (float)(_Float16)(a1 * kRsqrt128);
}

template <int K, int MR, bool PL, bool DIRECT>
__device__ __forceinline__ void fused_gateup(const FusedArgs& a, FusedShared<MR>& s, const Item& it, int item,
                                             int nb, int p) {
    constexpr int KBF = FusedShared<MR>::KBF;
    constexpr int KL = K > 0 ? K : 1;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int cnt = it.cnt;
    const int nbI = a.I / 128;
    const KRange kr = k_range(p, a.P_gu, a.H / 16);
    const int proj = wave >> 1, half = wave & 1;
    const uint32_t* tr = reinterpret_cast<const uint32_t*>(proj ? s.tab[3] : s.tab[0]);
    const int tn = a.I / 16;
    const size_t rs = (size_t)a.gu_tn * (8 * KL);
    const uint32_t* sp = tr + (size_t)nb * (64 * KL) + (size_t)kr.t0 * rs;
    StripRing<KL, kFusedRing> ring;

    // stage the blocks covering the k range of the item's x rows (16-byte loads; rows past cnt are zero) in xs[1]
    // and both input sign vectors in su. The loads are issued before the first weight rows (every address clamped
    // in range, no branch), so waiting for them does not wait for the weights.
    {
        constexpr int XI = (MR * KBF * 16 + 255) / 256, SI = (KBF * 128 + 255) / 256;
        const int k0 = kr.b0 * 128, nch = kr.kbs * 16;           // 16-byte chunks per row
        const uint16_t* sg = reinterpret_cast<const uint16_t*>(s.tab[1]) + k0;
        const uint16_t* su = reinterpret_cast<const uint16_t*>(s.tab[4]) + k0;
        u32x4_t xv[XI];
        uint16_t gv[SI], uv[SI];
#pragma unroll
        for (int j = 0; j < XI; ++j) {
            int c = threadIdx.x + 256 * j;
            c = c < MR * nch ? c : MR * nch - 1;
            const int m = c / nch, o = c - m * nch, mm = m < cnt ? m : 0;
            xv[j] = ldg(reinterpret_cast<const u32x4_t*>(a.x + (int64_t)(s.rows[mm] / a.slots) * a.x_ld + k0) + o);
        }
#pragma unroll
        for (int j = 0; j < SI; ++j) {
            int c = threadIdx.x + 256 * j;
            c = c < kr.kbs * 128 ? c : kr.kbs * 128 - 1;
            gv[j] = ldg(sg + c);
            uv[j] = ldg(su + c);
        }
        if (K > 0) strip_prefetch<KL, kFusedRing, false, PL>(sp, rs, half, kr.nt, 2, lane, ring);   // nt >= 8 > half
#pragma unroll
        for (int j = 0; j < XI; ++j) {
            const int c = threadIdx.x + 256 * j;
            if (c < MR * nch) {
                const int m = c / nch, o = c - m * nch;
                const u32x4_t z = {0u, 0u, 0u, 0u};
                *reinterpret_cast<u32x4_t*>(&s.xs[1][m][o * 8]) = m < cnt ? xv[j] : z;
            }
        }
#pragma unroll
        for (int j = 0; j < SI; ++j) {
            const int c = threadIdx.x + 256 * j;
            if (c < kr.kbs * 128) {
                s.su[0][c] = __builtin_bit_cast(_Float16, gv[j]);
                s.su[1][c] = __builtin_bit_cast(_Float16, uv[j]);
            }
        }
    }
    __syncthreads();
    // input transform of block (m, b) for both projections by one wave: xs[0] <- gate, xs[1] <- up (in place)
    for (int i = wave; i < cnt * kr.kbs; i += 4) {
        const int m = i / kr.kbs, b = i - m * kr.kbs;
        _Float16* xg = &s.xs[0][m][b * 128];
        _Float16* xu = &s.xs[1][m][b * 128];
        const float xa = (float)xu[lane], xb = (float)xu[lane + 64];
        float ga = (float)(_Float16)(xa * (float)s.su[0][b * 128 + lane]);
        float gb = (float)(_Float16)(xb * (float)s.su[0][b * 128 + lane + 64]);
        float ua = (float)(_Float16)(xa * (float)s.su[1][b * 128 + lane]);
        float ub = (float)(_Float16)(xb * (float)s.su[1][b * 128 + lane + 64]);
        fwht128_wave(ga, gb, lane);
        fwht128_wave(ua, ub, lane);
        xg[lane] = (_Float16)(ga * kRsqrt128);
        xg[lane + 64] = (_Float16)(gb * kRsqrt128);
        xu[lane] = (_Float16)(ua * kRsqrt128);
        xu[lane + 64] = (_Float16)(ub * kRsqrt128);
    }
    // rows past cnt are never read: the GEMV variant matches cnt (and reads row m < its size only)
    __syncthreads();
    range_sums(s, 2, cnt, kr, wave, lane);

    float acc[MR][2];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m][0] = acc[m][1] = 0.f;
    if (K > 0) {
        item_gemv<KL, MR, PL>(cnt, sp, rs, half, kr.nt, 2, lane, &s.xs[proj][0][kr.xo], KBF * 128, acc, ring);
    } else {
        const uint8_t* km = reinterpret_cast<const uint8_t*>(proj ? it.km[2] : it.km[0]);
        const int32_t* wo = reinterpret_cast<const int32_t*>(proj ? it.km[3] : it.km[1]);
        item_gemv_mixed<MR>(cnt, tr, km, wo, tn, nb * 8, kr.t0, half, kr.nt, 2, lane, &s.xs[proj][0][kr.xo],
                            KBF * 128, acc);
    }

#pragma unroll
    for (int m = 0; m < MR; ++m) {
        s.red[wave][m][0][lane] = acc[m][0];
        s.red[wave][m][1][lane] = acc[m][1];
    }
    __syncthreads();
    const int cbase = 16 * (lane >> 3) + (lane & 7);
    const size_t slot = (size_t)item * nbI + nb;
    if (half == 0) {
        for (int m = 0; m < cnt; ++m) {
            const float sx = s.ksum[proj][m];
            float* dst = a.part_gu + (((slot * a.P_gu + p) * 2 + proj) * MR + m) * 128;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float v = s.red[wave][m][h][lane] + s.red[wave + 1][m][h][lane];
                splitk_store(dst + cbase + 8 * h, kMul1C1 * v + kMul1C2 * sx);
            }
        }
    }
    if constexpr (DIRECT) {
        // the down jobs build their inputs from the partials themselves: publish this split to the item counter
        __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
        __syncthreads();
        if (threadIdx.x == 0) atomic_add_agent(&a.cnt_item[item * kCS], 1);
        return;
    }
    if (!splitk_arrive(&a.cnt_gu[slot * kCS], a.P_gu, &s.flag)) return;

    for (int m = wave; m < cnt; m += 4) {
        float r0, r1;
        down_input<MR>(a, s.tab, slot, nb, m, lane, r0, r1);
        float* dst = a.abuf + ((size_t)item * MR + m) * a.I + nb * 128;
        splitk_store(dst + lane, r0);
        splitk_store(dst + lane + 64, r1);
    }
    __builtin_amdgcn_s_waitcnt(0);      // this wave's down-input stores have completed
    __syncthreads();
    // P_gu + 1: block nb of the item's down input is published (its consumers count on from there and the last one
    // clears it)
    if (threadIdx.x == 0) atomic_add_agent(&a.cnt_gu[slot * kCS], 1);
}

// split of P over T tile-rows that holds tile-row t (splits start at floor(p T / P))
__device__ __forceinline__ int split_of(int t, int P, int T) {
    const int p = (int)(((int64_t)(t + 1) * P - 1) / T);
    return p < P - 1 ? p : P - 1;
}

template <int K, int MR, bool PL, bool DIRECT>
__device__ __forceinline__ void fused_down(const FusedArgs& a, FusedShared<MR>& s, uint64_t vm0, uint64_t vm1,
                                           const Item& it, int item, int nb, int p) {
    constexpr int KBF = FusedShared<MR>::KBF;
    constexpr int KL = K > 0 ? K : 1;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int cnt = it.cnt;
    const int nbI = a.I / 128, nbH = a.H / 128;
    const KRange kr = k_range(p, a.P_d, a.I / 16);
    const uint32_t* tr = reinterpret_cast<const uint32_t*>(s.tab[6]);
    const int tn = a.H / 16;
    const size_t rs = (size_t)tn * (8 * KL);
    const uint32_t* sp = tr + (size_t)nb * (64 * KL) + (size_t)kr.t0 * rs;
    StripRing<KL, kFusedRing> ring;
    if (K > 0) strip_prefetch<KL, kFusedRing, false, PL>(sp, rs, wave, kr.nt, 4, lane, ring);   // nt >= 8 > wave
    // the epilogue's output signs and row weights, loaded now so the epilogue waits for nothing
    constexpr int RW = (MR + 3) / 4;                     // rows m = wave + 4 j of this wave
    const uint16_t* svd = reinterpret_cast<const uint16_t*>(s.tab[8]) + nb * 128;
    const float sd0 = h2f(ldg(svd + lane)), sd1 = h2f(ldg(svd + lane + 64));
    float wrow[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) wrow[j] = pair_weight(a, s.rows[wave + 4 * j < MR ? wave + 4 * j : 0], s.rw);

    // wait for the down input this job reads and count the job as a consumer of its counter (the last consumer clears
    // it for the next call; every consumer passed its wait before it counts itself, so the last count comes after
    // every wait on the counter). Direct mode: every gate|up split of the item (nbI * P_gu arrivals on the item
    // counter), counted right after the wait. Otherwise: just the column blocks of I in this job's k range, each
    // published by its gate|up epilogue (counter P_gu + 1), so a down job starts as soon as its own blocks are in;
    // lane b of wave 0 watches block b0 + b, and its count is issued once the GEMV's accumulators are stored and
    // checked at the end of the job (consumer_done), off the job's path.
    auto counter_of = [&](int lane0) {
        return DIRECT ? &a.cnt_item[item * kCS]
                      : &a.cnt_gu[((size_t)item * nbI + kr.b0 + (lane0 < kr.kbs ? lane0 : 0)) * kCS];
    };
    if (threadIdx.x < 64) {
        const int lane0 = threadIdx.x;
        const bool mine = DIRECT ? lane0 == 0 : lane0 < kr.kbs;
        int* c = counter_of(lane0);
        const int need = DIRECT ? nbI * a.P_gu : a.P_gu + 1;
        int n = 0, back = 1;
        while (__ballot(mine && atomic_load_agent(c) < need)) {
            if (++n > a.spin_max) {
                if (lane0 == 0) report_timeout(a.status);
                break;
            }
            for (int z = 0; z < back; ++z) __builtin_amdgcn_s_sleep(2);
            back = back < 4 ? 2 * back : 4;
        }
        if (DIRECT && mine && atomic_add_agent(c, 1) == need + a.DN - 1) atomic_store_agent(c, 0);
    }
    __syncthreads();
    int cons_old = 0;                                    // per-block mode: this lane's count, issued after the GEMV
    auto consumer_done = [&]() {
        if constexpr (!DIRECT) {
            const int lane0 = threadIdx.x;
            if (lane0 < kr.kbs) {                        // lanes of wave 0 (kbs <= 64)
                // consumers of block bi: every column block of H times the k splits whose range touches it
                const int bi = kr.b0 + lane0, T = a.I / 16;
                const int last = a.P_gu + nbH * (split_of(8 * bi + 7, a.P_d, T) - split_of(8 * bi, a.P_d, T) + 1);
                if (cons_old == last) atomic_store_agent(counter_of(lane0), 0);
            }
        }
    };

    if constexpr (DIRECT) {
        // block (m, b) of the down input straight from the gate|up partials, one wave each
        for (int i = wave; i < cnt * kr.kbs; i += 4) {
            const int m = i / kr.kbs, b = i - m * kr.kbs, bi = kr.b0 + b;
            float r0, r1;
            down_input<MR>(a, s.tab, (size_t)item * nbI + bi, bi, m, lane, r0, r1);
            s.xs[0][m][b * 128 + lane] = (_Float16)r0;
            s.xs[0][m][b * 128 + lane + 64] = (_Float16)r1;
        }
    } else {
    // the wave's blocks (m, b) = (i / kbs, i % kbs), i = wave, wave + 4, ...: every load first, then convert
    constexpr int NBW = (MR * KBF + 3) / 4;
    float va[NBW], vb[NBW];
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        const int i = wave + 4 * j, m = i / kr.kbs, b = i - m * kr.kbs;
        const int mm = m < cnt ? m : 0;                  // unconditional load (rows past cnt read row 0, unused)
        const float* src = a.abuf + ((size_t)item * MR + mm) * a.I + (kr.b0 + b) * 128;
        va[j] = splitk_load(src + lane);
        vb[j] = splitk_load(src + lane + 64);
    }
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        const int i = wave + 4 * j, m = i / kr.kbs, b = i - m * kr.kbs;
        if (m < cnt) {
            s.xs[0][m][b * 128 + lane] = (_Float16)va[j];
            s.xs[0][m][b * 128 + lane + 64] = (_Float16)vb[j];
        }
    }
    }
    __syncthreads();
    range_sums(s, 1, cnt, kr, wave, lane);

    float acc[MR][2];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m][0] = acc[m][1] = 0.f;
    if (K > 0) {
        item_gemv<KL, MR, PL>(cnt, sp, rs, wave, kr.nt, 4, lane, &s.xs[0][0][kr.xo], KBF * 128, acc, ring);
    } else {
        const uint8_t* km = reinterpret_cast<const uint8_t*>(it.km[4]);
        const int32_t* wo = reinterpret_cast<const int32_t*>(it.km[5]);
        item_gemv_mixed<MR>(cnt, tr, km, wo, tn, nb * 8, kr.t0, wave, kr.nt, 4, lane, &s.xs[0][0][kr.xo],
                            KBF * 128, acc);
    }

#pragma unroll
    for (int m = 0; m < MR; ++m) {
        s.red[wave][m][0][lane] = acc[m][0];
        s.red[wave][m][1][lane] = acc[m][1];
    }
    __syncthreads();
    if (!DIRECT && threadIdx.x < kr.kbs) cons_old = atomic_add_agent(counter_of(threadIdx.x), 1);
    const int cbase = 16 * (lane >> 3) + (lane & 7);
    const size_t slot = (size_t)item * nbH + nb;
    const bool split = a.P_d > 1;
    if (wave == 0) {
        for (int m = 0; m < cnt; ++m) {
            const float sx = s.ksum[0][m];
            float* dst = a.part_d + ((slot * a.P_d + p) * MR + m) * 128;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float v = kMul1C1 * (s.red[0][m][h][lane] + s.red[1][m][h][lane] + s.red[2][m][h][lane] +
                                           s.red[3][m][h][lane]) + kMul1C2 * sx;
                if (split) splitk_store(dst + cbase + 8 * h, v);
                else s.cv[m][cbase + 8 * h] = v;
            }
        }
    }
    if (split) {
        if (!splitk_arrive(&a.cnt_d[slot * kCS], a.P_d, &s.flag)) {
            consumer_done();
            return;
        }
    } else {
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int m = wave + 4 * j;
        if (m >= cnt) break;
        const int pr = s.rows[m];
        const float w = wrow[j];
        float v0, v1;
        if (split) {
            const int off[2] = {m * 128 + lane, m * 128 + lane + 64};
            float v[2];
            sum_partials<2>(a.part_d + slot * a.P_d * MR * 128, MR * 128, off, a.P_d, v);
            v0 = v[0];
            v1 = v[1];
        } else {
            v0 = s.cv[m][lane];
            v1 = s.cv[m][lane + 64];
        }
        fwht128_wave(v0, v1, lane);
        const float y0 = v0 * kRsqrt128 * sd0 * w, y1 = v1 * kRsqrt128 * sd1 * w;
        if (!DIRECT && a.slots == 1) {
            // one slot per token (a dense MLP, which runs in per-block mode): the token's output block is this row,
            // as the combine would sum it (0 + y: the same bits), written here without the y round trip and the
            // token count (the direct-mode instantiations leave this out: one-token decode layers measured it slower)
            const int t = pr;
            const int c0 = nb * 128 + lane, c1 = c0 + 64;
            if (a.out_f32) {
                float* o = reinterpret_cast<float*>(a.out) + (int64_t)t * a.out_ld;
                o[c0] = 0.f + y0;
                o[c1] = 0.f + y1;
            } else {
                uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + (int64_t)t * a.out_ld;
                o[c0] = f2h(0.f + y0);
                o[c1] = f2h(0.f + y1);
            }
            continue;
        }
        float* dst = a.y + (size_t)pr * a.H + nb * 128;
        splitk_store(dst + lane, y0);
        splitk_store(dst + lane + 64, y1);
    }
    if (split && threadIdx.x == 0) a.cnt_d[slot * kCS] = 0;

    // combine: count this item's rows into their tokens; finish the tokens whose slots are now all in (with one slot
    // per token the rows were written above)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < cnt) {                 // lane m counts row m (rows of one item belong to different tokens)
        const int m = threadIdx.x;
        const int t = s.rows[m] / a.slots;
        const int nv = popc_range(vm0, vm1, t * a.slots, a.slots);
        const bool written = !DIRECT && a.slots == 1;
        const int old = written ? 0 : atomic_add_agent(&a.cnt_tok[((size_t)t * nbH + nb) * kCS], 1);
        s.comb[m] = (!written && old == nv - 1) ? t : -1;
    }
    __syncthreads();
    for (int m = wave; m < cnt; m += 4) {
        const int t = s.comb[m];
        if (t < 0) continue;
        const int c0 = nb * 128 + lane, c1 = c0 + 64;
        float v0 = 0.f, v1 = 0.f;
        // slots in order, 8 at a time: every load of a group issued before the first add (invalid slots read a
        // valid row and add zero)
        for (int j0 = 0; j0 < a.slots; j0 += 8) {
            float y0[8], y1[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int jj = j0 + j < a.slots ? j0 + j : a.slots - 1;
                const float* yr = a.y + (size_t)(t * a.slots + jj) * a.H;
                y0[j] = splitk_load(yr + c0);
                y1[j] = splitk_load(yr + c1);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int pr = t * a.slots + j0 + j;
                const bool ok = j0 + j < a.slots && (((pr < 64 ? vm0 >> pr : vm1 >> (pr - 64))) & 1);
                v0 += ok ? y0[j] : 0.f;
                v1 += ok ? y1[j] : 0.f;
            }
        }
        if (a.out_f32) {
            float* o = reinterpret_cast<float*>(a.out) + (int64_t)t * a.out_ld;
            o[c0] = v0;
            o[c1] = v1;
        } else {
            uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + (int64_t)t * a.out_ld;
            o[c0] = f2h(v0);
            o[c1] = f2h(v1);
        }
        if (lane == 0) a.cnt_tok[((size_t)t * nbH + nb) * kCS] = 0;
    }
    consumer_done();
}

// Wave issue priority 0..3 (s_setprio takes an immediate).
__device__ __forceinline__ void set_wave_priority(int p) {
    if (p <= 0) __builtin_amdgcn_s_setprio(0);
    else if (p == 1) __builtin_amdgcn_s_setprio(1);
    else if (p == 2) __builtin_amdgcn_s_setprio(2);
    else __builtin_amdgcn_s_setprio(3);
}

// KG: bits of gate and up, KD: bits of down (equal, or both 0 for per-tile K); PL: weights in PLANAR4 word order.
// DIRECT: the down jobs build their inputs from the gate|up partials (FusedArgs::direct; one instantiation per mode,
// so that neither carries the other's code and registers).
template <int KG, int KD, int MR, bool PL, bool DIRECT>
__global__ __launch_bounds__(256) void moe_fused_kernel(FusedArgs a) {
    __shared__ __attribute__((aligned(16))) FusedShared<MR> s;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = blockIdx.x;
    const int gi = g / a.GU, gr0 = g - gi * a.GU;
    // one row per item with in-layer routing: item i is pair i (pair_item), described by every wave; otherwise wave 0
    // groups the pairs and describes the gate|up job's item while the others wait at the barrier
    const bool by_pair = MR == 1 && a.logits && (a.slots == a.topk || (unsigned)a.shared < (unsigned)a.E);
    if (a.logits) {
        if (by_pair && a.M > 1) {
            // just the tokens of this workgroup's items: its gate|up item's (wave 0) and its down item's (wave 1); the
            // workgroup whose gate|up item is a token's first pair writes that token's picks out
            const int tg = g < a.J_gu && gi < a.np ? gi / a.slots : -1;
            const int td = gi >= 1 && gi - 1 < a.np && gr0 < a.DN ? (gi - 1) / a.slots : -1;
            if (wave == 0 && tg >= 0) route_token(a, tg, lane, s.rid, s.rw, gr0 == 0 && gi == tg * a.slots);
            if (wave == 1 && td >= 0 && td != tg) route_token(a, td, lane, s.rid, s.rw, false);
        } else {
            route_in_layer(a, wave, lane, s.rid, s.rw);
        }
        __syncthreads();
    }
    Groups gr;
    int nitems;
    uint64_t v0, v1;
    if (by_pair) {
        nitems = a.np;
        v0 = a.np >= 64 ? ~0ull : (1ull << a.np) - 1;
        v1 = a.np <= 64 ? 0ull : a.np >= 128 ? ~0ull : (1ull << (a.np - 64)) - 1;
        if constexpr (MR == 1)
            if (g < a.J_gu && gi < nitems) pair_item<KG>(a, gi, lane, s);
    } else {
        if (wave == 0) {
            group_pairs<MR>(a, lane, gr, s.ge, s.rid);
            if (lane == 0) {
                s.valid[0] = gr.v0;
                s.valid[1] = gr.v1;
                s.nitems = gr.nitems;
            }
            if (g < a.J_gu && gi < gr.nitems) item_info<KG, MR>(a, gr, gi, lane, s);
        }
        __syncthreads();
        nitems = s.nitems;
        v0 = s.valid[0];
        v1 = s.valid[1];
    }
    if (g == 0) {
        // tokens with no valid slot get a zero output row
        for (int tk = 0; tk < a.M; ++tk) {
            if (popc_range(v0, v1, tk * a.slots, a.slots)) continue;
            for (int c = threadIdx.x; c < a.H; c += 256) {
                if (a.out_f32) reinterpret_cast<float*>(a.out)[(int64_t)tk * a.out_ld + c] = 0.f;
                else reinterpret_cast<uint16_t*>(a.out)[(int64_t)tk * a.out_ld + c] = 0;
            }
        }
    }
    // Issue priority: a CU's SIMDs pick the oldest wave among equals, so without priorities the gate|up jobs of the
    // last items (the youngest workgroups) finish last and hold back their down jobs, the end of the layer. Gate|up
    // jobs run at 1..3 rising with the item number and down jobs at 0 (C3 at 4 tokens: 38.1 us against 39.9).
    set_wave_priority(1 + (3 * gi) / (nitems > 0 ? nitems : 1));
    if (g < a.J_gu && gi < nitems)
        fused_gateup<KG, MR, PL, DIRECT>(a, s, read_item<KG, MR>(s), gi, gr0 / a.P_gu, gr0 % a.P_gu);
    // the down jobs of the previous item (uniform branch)
    const int di = gi - 1;
    if (di < 0 || di >= nitems || gr0 >= a.DN) return;
    __syncthreads();                    // the gate|up job's LDS (rows, tab, xs) is free again
    if (by_pair) {
        if constexpr (MR == 1) pair_item<KD>(a, di, lane, s);
    } else {
        if (wave == 0) item_info<KG, MR>(a, gr, di, lane, s);
        __syncthreads();
    }
    set_wave_priority(0);
    const Item it = read_item<KG, MR>(s);
    for (int r = gr0; r < a.DN; r += a.GU) {
        // k-split major: the down jobs reading the first column blocks of I (published first) come first
        fused_down<KD, MR, PL, DIRECT>(a, s, v0, v1, it, di, r % (a.H / 128), r / (a.H / 128));
        __syncthreads();
    }
}

typedef void (*fused_fn)(FusedArgs);

// Mixed-bitrate instantiations (gate/up K != down K), exl3_moe_fused_mixed.hip; nullptr when not built.
fused_fn pick_fused_mixed(int Kg, int Kd, int MR, bool direct);
// PLANAR4 instantiations (K = 3, 5, 6, 7), exl3_moe_fused_planar.hip; nullptr for other K.
fused_fn pick_fused_planar(int K, int MR, bool direct);

}  // namespace exl3
