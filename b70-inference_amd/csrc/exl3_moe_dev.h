// Device helpers shared by the GEMV and MFMA MoE kernels.
#pragma once

#include "exl3_device.h"
#include "exl3_gemv.h"
#include "exl3_moe.h"
#include "../../include/exl3mi.h"

namespace exl3 {

// Gated activation in fp32. SiLU: min(silu(g), L) * clamp(u, -L, L) (L = 0: no clamp, ext-op-inventory.md:944-956).
// GELU-tanh: 0.5 g (1 + tanh(z)) * u evaluated as g * sigmoid(2z) * u (no cancellation for negative g).
__device__ __forceinline__ float act_mul_dev(float g, float u, int act, float L) {
    if (act == EXL3_ACT_GELU_TANH) {
        const float z2 = 1.5957691216057308f * (g + 0.044715f * g * g * g);   // 2 sqrt(2 / pi) (g + 0.044715 g^3)
        return g / (1.f + expf(-z2)) * u;
    }
    float s = g / (1.f + expf(-g));
    if (L > 0.f) {
        s = fminf(s, L);
        u = fminf(fmaxf(u, -L), L);
    }
    return s * u;
}

// out[t, 128-column block nb] = sum over t's slots in slot order of y[pair] (fp32); resets the token's counter.
// Called by one wave once every slot of token t has published its y row (agent-scope loads see them).
__device__ __forceinline__ void combine_token(const MoeArgs& a, int t, int nb, int lane) {
    const int c0 = nb * 128 + lane, c1 = c0 + 64;
    float v0 = 0.f, v1 = 0.f;
    // slots in order, 8 at a time: every load of a group issued before the first add (a missing slot reads pair 0's
    // row and adds zero)
    for (int j0 = 0; j0 < a.slots; j0 += 8) {
        int pr[8];
        float y0[8], y1[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) pr[j] = j0 + j < a.slots ? a.pair_of[t * a.slots + j0 + j] : -1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float* y = a.y + (size_t)(pr[j] >= 0 ? pr[j] : 0) * a.H;
            y0[j] = splitk_load(y + c0);
            y1[j] = splitk_load(y + c1);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v0 += pr[j] >= 0 ? y0[j] : 0.f;
            v1 += pr[j] >= 0 ? y1[j] : 0.f;
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
    if (lane == 0) a.cnt_tok[(size_t)t * (a.H / 128) + nb] = 0;
}

template <int V, int SC>
__device__ __forceinline__ void route_select(const uint32_t (&key)[V], const float (&g)[V], float mx, float sum, int k,
                                             int lane, bool renorm, float scaling, int& id, float& w);

// Top-k routing of one row by one wave. Scoring SC (EXL3_SCORE_*), per entry with logit f and bias b (0 without one):
//   softmax (trellis-serve.patch:395-441): rank by f + b; weight source g = f + b (bias_both) or f (selection-only
//            bias, the reference's `cold` term); p = exp(g - max g) / sum exp(g - max g) over the row
//   sigmoid (routing_ds3_nogroup, glm/xpu/glm_xpu/ops.py:177-193): s = sigmoid(f); rank by s + b, or by f without a
//            bias; weight source s
//   sqrt-softplus (dsv41/xpu/csrc/dsv_moe_glue.sycl:155-193): s = sqrt(softplus(f)) (f itself above 20); rank by s + b;
//            weight source s
// Exact ties rank to the lower index. The k picks' weights are w = v * scaling / (sum of picked v + 1e-20) with
// renorm, v * scaling without (v = p or s). Lane l keeps the order keys of entries l + 64 v (v < V, E <= 64 V) in
// registers; picked and padding entries hold key 0, NaN keys 1 (below every number, still pickable, as a stable
// descending sort places them last). Each round is one DPP wave max, a ballot of the lanes holding it, and a DPP wave
// min of their lowest indices only when several lanes tie. Lane j < k returns pick j in (id, w).
//
// ADJ (sigmoid and sqrt-softplus only): the picks rank by s * mul + b + max(res, -1e30) instead (mul, res per entry,
// either may be null: the reference dsv router's residency terms, dsv41/xpu/csrc/dsv_moe_glue.sycl:155-193), each
// operation rounded separately; the weights still come from s.
template <int V, int SC, bool ADJ = false>
__device__ __forceinline__ void route_row(const float* __restrict__ z, const float* __restrict__ bias, int E, int k,
                                          int lane, bool bias_both, bool renorm, float scaling, int& id, float& w,
                                          const float* __restrict__ mul = nullptr,
                                          const float* __restrict__ res = nullptr) {
    // every load issued before any is used (clamped indices, no per-element branch): one memory round trip
    float f[V], b[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int i = lane + 64 * v;
        f[v] = ldg(z + (i < E ? i : E - 1));
    }
    if (bias) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int i = lane + 64 * v;
            b[v] = ldg(bias + (i < E ? i : E - 1));
        }
    }
    float mv[V], rv[V];
    if (ADJ) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int i = lane + 64 * v < E ? lane + 64 * v : E - 1;
            mv[v] = mul ? ldg(mul + i) : 1.f;
            rv[v] = res ? ldg(res + i) : 0.f;
        }
    }
    float g[V];                          // weight source per entry
    uint32_t key[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        float r;
        if (SC == EXL3_SCORE_SOFTMAX) {
            r = bias ? f[v] + b[v] : f[v];
            g[v] = bias_both ? r : f[v];
        } else {
            float s;
            if (SC == EXL3_SCORE_SIGMOID) {
                s = 1.f / (1.f + expf(-f[v]));
            } else {
                s = sqrtf(f[v] > 20.f ? f[v] : log1pf(expf(f[v])));
            }
            g[v] = s;
            r = bias ? s + b[v] : (SC == EXL3_SCORE_SIGMOID ? f[v] : s);
        }
        if (ADJ && SC != EXL3_SCORE_SOFTMAX) {
            r = __fmul_rn(g[v], mv[v]);
            if (bias) r = __fadd_rn(r, b[v]);
            if (res) r = __fadd_rn(r, fmaxf(rv[v], -1e30f));
        }
        const int i = lane + 64 * v;
        key[v] = i < E ? (r != r ? 1u : float_key(r)) : 0u;
    }
    // softmax denominators: renormalised weights need only the picks (w = exp(g - m) / sum over the picks of
    // exp(g - m), m the largest picked g: the full softmax denominator cancels, route_select); a NaN anywhere in the
    // row still makes every weight NaN, as the full softmax does. Unrenormalised weights need the full sum.
    float mx = 0.f, sum = 1.f;
    if (SC == EXL3_SCORE_SOFTMAX) {
        if (renorm) {
            bool ln = false;
#pragma unroll
            for (int v = 0; v < V; ++v) ln = ln || (lane + 64 * v < E && g[v] != g[v]);
            sum = __ballot(ln) ? __builtin_nanf("") : 1.f;
        } else {
            uint32_t lmax = 0u;
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const int i = lane + 64 * v;
                lmax = max(lmax, i < E ? (g[v] != g[v] ? 1u : float_key(g[v])) : 0u);
            }
            mx = key_float(wave_max_u32(lmax));
            float se = 0.f;
#pragma unroll
            for (int v = 0; v < V; ++v)
                if (lane + 64 * v < E) se += expf(g[v] - mx);
            sum = wave_sum_f32(se);
        }
    }

    route_select<V, SC>(key, g, mx, sum, k, lane, renorm, scaling, id, w);
}

// A lane's two best keys not yet picked, ascending v so that equal keys keep their lowest index first: (k1, v1, g1)
// then (k2, v2, g2); key 0 means none. A lane's picks come in descending (key, ascending v) order, so the keys not yet
// picked are those ordered after its last pick (kl, vl); vl < 0: nothing picked yet.
template <int V>
__device__ __forceinline__ void lane_top2(const uint32_t (&key)[V], const float (&g)[V], uint32_t kl, int vl,
                                          uint32_t& k1, int& v1, float& g1, uint32_t& k2, int& v2, float& g2) {
    k1 = k2 = 0u;
    v1 = v2 = 0;
    g1 = g2 = 0.f;
    // selects only (no branch per key: each would switch the exec mask on the routing's dependency chain)
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const bool left = vl < 0 || key[v] < kl || (key[v] == kl && v > vl);
        const uint32_t kv = left ? key[v] : 0u;
        const bool gt1 = kv > k1, gt2 = kv > k2;
        const uint32_t nk2 = gt1 ? k1 : (gt2 ? kv : k2);
        const int nv2 = gt1 ? v1 : (gt2 ? v : v2);
        const float ng2 = gt1 ? g1 : (gt2 ? g[v] : g2);
        k1 = gt1 ? kv : k1;
        v1 = gt1 ? v : v1;
        g1 = gt1 ? g[v] : g1;
        k2 = nk2;
        v2 = nv2;
        g2 = ng2;
    }
}

// The k rounds of route_row over prepared order keys (0: not pickable) and weight sources: lane j < k returns pick j
// in (id, w); mx / sum are the softmax maximum and denominator (SC softmax only). Each round takes the wave maximum of
// the lanes' best remaining keys (ties: the lowest index) from a per-lane cache of two; a lane rescans its keys only
// when a pick empties its cache, so a round costs a wave reduction rather than a scan of every key.
template <int V, int SC>
__device__ __forceinline__ void route_select(const uint32_t (&key)[V], const float (&g)[V], float mx, float sum, int k,
                                             int lane, bool renorm, float scaling, int& id, float& w) {
    float gv = 0.f;
    id = -1;
    uint32_t kl = 0u, k1, k2;
    int vl = -1, v1, v2;
    float g1, g2;
    lane_top2<V>(key, g, kl, vl, k1, v1, g1, k2, v2, g2);
    for (int j = 0; j < k; ++j) {
        const uint32_t kmax = wave_max_u32(k1);
        if (kmax == 0u) break;            // fewer than k entries (k <= E is checked on the host)
        const uint64_t mask = __ballot(k1 == kmax);
        int wl = __ffsll((unsigned long long)mask) - 1;
        if (__popcll(mask) != 1) wl = (int)(wave_min_u32(k1 == kmax ? (uint32_t)(lane + 64 * v1) : 0xFFFFFFFFu) & 63u);
        const int vw = __builtin_amdgcn_readlane(v1, wl);
        const float gw = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, g1), wl));
        const bool empty = __builtin_amdgcn_readlane((int)k2, wl) == 0;
        // the winner's cache moves up one entry; selects rather than a branch on the lane, so that no exec-mask
        // switch sits on the round's dependency chain
        const bool win = lane == wl;
        kl = win ? k1 : kl;
        vl = win ? v1 : vl;
        k1 = win ? k2 : k1;
        v1 = win ? v2 : v1;
        g1 = win ? g2 : g1;
        k2 = win ? 0u : k2;
        id = lane == j ? wl + 64 * vw : id;
        gv = lane == j ? gw : gv;
        if (empty) lane_top2<V>(key, g, kl, vl, k1, v1, g1, k2, v2, g2);   // uniform: the winner's cache is empty
    }
    float p;
    if (SC == EXL3_SCORE_SOFTMAX && renorm) {
        // exp relative to the largest picked g (sum is 1, or NaN when the row holds a NaN)
        const uint32_t lk = id >= 0 ? (gv != gv ? 1u : float_key(gv)) : 0u;
        const float mp = key_float(wave_max_u32(lk));
        p = id >= 0 ? expf(gv - mp) * sum : 0.f;
    } else {
        p = id >= 0 ? (SC == EXL3_SCORE_SOFTMAX ? expf(gv - mx) / sum : gv) : 0.f;
    }
    const float s = wave_sum_f32(p);
    w = renorm ? p * scaling / (s + 1e-20f) : p * scaling;
}

}  // namespace exl3
