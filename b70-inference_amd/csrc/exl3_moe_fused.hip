// Fused small-batch MoE layer: host side (eligibility, grid and split sizing, workspace, launch). The kernel and its
// device code are in exl3_moe_fused.h; gate/up and down bitrates that differ are instantiated in
// exl3_moe_fused_mixed.hip.
#include "exl3_moe_fused.h"

namespace exl3 {


template <int MR, bool D>
static fused_fn pick_fused_d(int K) {
    switch (K) {
        case 0: return moe_fused_kernel<0, 0, MR, false, D>;
        case 1: return moe_fused_kernel<1, 1, MR, false, D>;
        case 2: return moe_fused_kernel<2, 2, MR, false, D>;
        case 3: return moe_fused_kernel<3, 3, MR, false, D>;
        case 4: return moe_fused_kernel<4, 4, MR, false, D>;
        case 5: return moe_fused_kernel<5, 5, MR, false, D>;
        case 6: return moe_fused_kernel<6, 6, MR, false, D>;
        case 7: return moe_fused_kernel<7, 7, MR, false, D>;
        default: return moe_fused_kernel<8, 8, MR, false, D>;
    }
}

// The instantiation for (gate/up K, down K, rows per item, word order, down-input mode); nullptr when not built.
static fused_fn pick_fused(const MoeArgs& m, int MR, bool direct) {
    if (m.planar) return pick_fused_planar(m.Kg, MR, direct);
    if (m.Kg != m.Kd) return pick_fused_mixed(m.Kg, m.Kd, MR, direct);
    switch (MR) {
        case 1: return direct ? pick_fused_d<1, true>(m.Kg) : pick_fused_d<1, false>(m.Kg);
        case 2: return direct ? pick_fused_d<2, true>(m.Kg) : pick_fused_d<2, false>(m.Kg);
        case 4: return direct ? pick_fused_d<4, true>(m.Kg) : pick_fused_d<4, false>(m.Kg);
        default: return direct ? pick_fused_d<8, true>(m.Kg) : pick_fused_d<8, false>(m.Kg);
    }
}

// largest number of 128-blocks that one of P tile-row splits of T tile-rows touches
static int max_staged_blocks(int P, int T) {
    int mx = 0;
    for (int p = 0; p < P; ++p) {
        const int t0 = (int)((int64_t)p * T / P), t1 = (int)((int64_t)(p + 1) * T / P);
        const int n = ((t1 + 7) >> 3) - (t0 >> 3);
        mx = n > mx ? n : mx;
    }
    return mx;
}

// k-split count: `want` clamped to [1, T / 8] (jobs of at least 8 tile-rows), raised until every split's staged blocks
// fit the kbf LDS blocks
static int fused_splits(int want, int T, int kbf) {
    int P = want;
    const int pmax = T / 8 > 1 ? T / 8 : 1;
    P = P < 1 ? 1 : (P > pmax ? pmax : P);
    while (P < T && max_staged_blocks(P, T) > kbf) ++P;
    return P;
}

// Eligible: gate, up and down share one K (or all per-tile), or down has one or two bits more than gate/up; at most
// kFusedMaxRows tokens and kFusedMaxPairs pairs; x rows 16-byte aligned.
bool moe_fused_ok(const MoeArgs& a) {
    return (a.Kg == a.Kd || pick_fused_mixed(a.Kg, a.Kd, 1, false) != nullptr) && (!a.planar || a.Kg == a.Kd) &&
           a.M <= kFusedMaxRows &&
           (int64_t)a.M * a.slots <= kFusedMaxPairs &&
           aligned(a.x, 16) && a.x_ld % 8 == 0 && env_int("EXL3MI_NO_FUSED", 0) == 0;
}

// Expected items of a batch at `mr` rows per item, routing taken as uniform: the routed experts' row counts are
// Binomial(M, p) with p = routed picks per token / routed experts, an item per started group of mr rows; a shared
// expert takes every token.
double moe_expected_items(const MoeArgs& m, int mr) {
    const bool sh = (unsigned)m.shared < (unsigned)m.E;
    const int routed_e = sh ? m.E - 1 : m.E, picks = sh ? m.slots - 1 : m.slots;
    double items = sh ? (double)((m.M + mr - 1) / mr) : 0.0;
    if (routed_e <= 0 || picks <= 0) return items;
    const double p = picks >= routed_e ? 1.0 : (double)picks / routed_e;
    double pmf = std::pow(1.0 - p, m.M), e_groups = 0.0;      // P(X = 0), then P(X = x) by the ratio recurrence
    for (int x = 1; x <= m.M; ++x) {
        pmf = p >= 1.0 ? (x == m.M ? 1.0 : 0.0) : pmf * (double)(m.M - x + 1) / x * p / (1.0 - p);
        e_groups += pmf * ((x + mr - 1) / mr);
    }
    return items + routed_e * e_groups;
}

// The smallest rows per item (1, 2, 4, 8 up to `cap`) at which every gate|up job of the expected items, each item
// split to its full k-split count, fits the device's resident grid for that instantiation (10 % slack), or 0 when
// none does. Wider items hold more registers and LDS (5 / 4 / 4 / 3 workgroups per CU at 1 / 2 / 4 / 8 rows) and
// run each tile-row longer; narrower items repeat an expert's decode for each group of rows. With the whole batch
// resident the narrowest width that fits wins: dense routing over experts of 2048 -> 512 (24 jobs per item), 8 tokens:
// 8 experts top-8 40.4 (eight rows) -> 28.8 us (two), 16 experts top-8 36.0 -> 32.1; 16 tokens: 8 experts top-2
// 35.8 -> 23.8 (one), 16 experts top-8 42.4 -> 37.8 (four), 32 experts top-8 44.1 -> 38.2 (four).
// Expected gate|up jobs of the batch at `mr` rows per item, each item split to its full k-split count, over the
// workgroups the device holds at once for that instantiation (0 when it is not built).
static int fused_load(const MoeArgs& m, int mr, double* load) {
    *load = 0.0;
    fused_fn fn = pick_fused(m, mr, false);
    if (!fn) return EXL3_OK;
    int resident = 0;
    const int rc = resident_blocks(reinterpret_cast<const void*>(fn), 256, &resident);
    if (rc) return rc;
    const int full = m.H / 16 / kFusedMinJobRows > 1 ? m.H / 16 / kFusedMinJobRows : 1;
    const int P = fused_splits(full, m.H / 16, mr <= 4 ? 8 : 4);
    *load = moe_expected_items(m, mr) * (m.I / 128) * P / (resident > 0 ? resident : 1);
    return EXL3_OK;
}

static int fused_fits(const MoeArgs& m, int mr, bool* fits) {
    double load = 0.0;
    const int rc = fused_load(m, mr, &load);
    *fits = load > 0.0 && load <= 1.1;
    return rc;
}

static int fused_fit_rows(const MoeArgs& m, int cap, int* out) {
    *out = 0;
    for (int mr = 1; mr <= cap; mr *= 2) {
        bool fits = false;
        const int rc = fused_fits(m, mr, &fits);
        if (rc) return rc;
        if (fits) {
            *out = mr;
            return EXL3_OK;
        }
    }
    return EXL3_OK;
}

// Rows per item for the batch (1, 2, 4 or 8).
static int fused_rows(const MoeArgs& m, int* out) {
    // rows per item: one when the routing is sparse (pairs <= E / 2: an expert rarely takes two rows, and the
    // one-row instantiation is the fastest; 512 experts of 2048 -> 512, top-10: 2 / 4 / 8 / 12 tokens 27.7 -> 25.8,
    // 36.2 -> 33.8, 54.5 -> 47.1, 68.3 -> 63.3 us against two rows per item; 64 experts, top-8, 4 tokens 28.8 -> 25.5);
    // otherwise the narrowest width whose jobs all fit the resident grid (fused_fit_rows), else up to the batch size
    // capped by the rows an expert takes on average (at most one: two rows per item, 64 experts, top-8, 8 tokens 34.0
    // against 36.6 with eight; experts of 4096 -> 1536 or wider fill the device at any width and take the fewest
    // items: 8 experts top-8, 8 tokens 52.6 us at eight rows, 63.0 at four; a dense MLP, one expert, takes every row)
    int MR = m.M <= 1 ? 1 : m.M <= 2 ? 2 : m.M <= 4 ? 4 : 8;
    const int64_t pairs = (int64_t)m.M * m.slots;
    if (pairs * 2 <= m.E) {
        // sparse: one row per item, unless the one-row jobs fill more than three resident grids (the layer then runs
        // at the device's throughput) and two-row items save a twentieth of the items: wide experts near E / 2
        // pairs, 8 experts of 4096 -> 14336, top-2, 2 tokens 95.5 -> 90.3 us, 16 experts at 4 tokens 173 -> 158;
        // 256 experts of 7168 -> 2048 and a shared expert, 4 tokens, whose shared rows pair up (9 % fewer items):
        // 440 -> 407. Below that load the one-row instantiation wins even with fewer items at two rows: C3 at
        // 8 tokens (1.5 grids, 7 % fewer items) 42 us at one row against 50 at two.
        const int cap = MR;
        MR = 1;
        double load1 = 0.0;
        int rc = 0;
        if (cap >= 2 && (rc = fused_load(m, 1, &load1))) return rc;
        if (cap >= 2 && load1 > 3.0 && moe_expected_items(m, 2) <= 0.95 * moe_expected_items(m, 1)) MR = 2;
    } else {
        int rc = 0, fit = 0;
        if ((rc = fused_fit_rows(m, MR, &fit))) return rc;
        if (fit) {
            MR = fit;
        } else {
            const int64_t rpe = (pairs + m.E - 1) / m.E;
            const int cap = rpe <= 1 ? 2 : rpe <= 2 ? 4 : 8;
            const int mcap = MR;
            if (MR > cap) MR = cap;
            // jobs of more than four resident grids: the layer runs at the device's throughput, so the width with
            // the fewest items per unit of per-item cost wins (128 experts of 4096 -> 1536, top-8, 16 tokens: 270 us
            // at two rows, 253 at four; per-item cost relative to two rows, from it: 0.81 / 1 / 1.02 / 1.27)
            double load = 0.0;
            if ((rc = fused_load(m, MR, &load))) return rc;
            if (load > 4.0) {
                static const double wt[4] = {0.81, 1.0, 1.02, 1.27};
                double best = 0.0;
                for (int mr = 1, q = 0; mr <= mcap; mr *= 2, ++q) {
                    const double c = moe_expected_items(m, mr) * wt[q];
                    if (pick_fused(m, mr, false) && (best == 0.0 || c < best)) {
                        best = c;
                        MR = mr;
                    }
                }
            }
        }
    }
    const int mr_env = env_int("EXL3MI_FUSED_MR", 0);
    if (mr_env == 1 || mr_env == 2 || mr_env == 4 || mr_env == 8) MR = mr_env;
    *out = MR;
    return EXL3_OK;
}

// Whether the fused layer takes the batch: eligible (moe_fused_ok), and its gate|up jobs at the chosen rows per item
// fill at most four resident grids. Past that the layer runs at the device's throughput and the multi-launch GEMV
// path is faster (fused against multi-launch: 129 experts of 4096 -> 1408 with a shared one, top-8, 4 / 8 / 14
// tokens 104.5 / 162.6 / 236 against 93.7 / 139.2 / 204 us; 256 experts of 7168 -> 2048 at per-tile K with a shared
// one, 2 / 4 / 8 tokens 251 / 406 / 746 against 217 / 375 / 683; 160 experts of 5120 -> 1536, 8 tokens 200.5 against
// 182), while below it the fused layer's shorter chain wins (the same 129 experts at 1 / 2 tokens 38 / 50 against
// 40.8 / 59.5; 128 experts of 2048 -> 768 at 4 / 8 tokens 35.2 / 49.5 against 43 / 62.3; C3). With 16 experts or
// fewer the fused layer keeps batches up to twelve grids (8 experts of 4096 -> 14336, top-2, 4 / 8 tokens 134.3 /
// 179 against 138.9 / 187; 16 tokens, 14 grids, 275.6 against 264). EXL3MI_FUSED_ALWAYS=1 takes every eligible
// batch, EXL3MI_FUSED_DECLINE=1 none.
bool moe_fused_take(const MoeArgs& m) {
    if (!moe_fused_ok(m) || env_int("EXL3MI_FUSED_DECLINE", 0)) return false;
    if (env_int("EXL3MI_FUSED_ALWAYS", 0)) return true;
    int MR = 1;
    double load = 0.0;
    if (fused_rows(m, &MR) || fused_load(m, MR, &load)) return true;   // errors surface on the fused path itself
    return !(load > 4.0 && (m.E > 16 || load > 12.0));
}

int moe_fused_path(const MoeArgs& m, hipStream_t st) {
    FusedArgs a{};
    if (m.uniform) {
        a.uniform = 1;
        for (int i = 0; i < 9; ++i) {
            a.tb[i] = m.tb[i];
            a.ts[i] = m.ts[i];
        }
    }
    a.x = m.x;
    a.x_ld = m.x_ld;
    a.gu_tn = m.gu_tn;
    a.M = m.M;
    a.H = m.H;
    a.I = m.I;
    a.topk = m.topk;
    a.slots = m.slots;
    a.E = m.E;
    a.shared = m.shared;
    a.np = m.M * m.slots;
    a.ids = m.ids;
    a.tw = m.tw;
    if (m.logits) {
        a.logits = m.logits;
        a.lg_ld = m.lg_ld;
        a.n_logits = m.n_logits;
        a.rbias = m.rbias;
        a.ids_out = m.ids_out;
        a.tw_out = m.tw_out;
    }
    a.tables = m.tables;
    a.kmaps = m.kmaps;
    a.act = m.act;
    a.limit = m.limit;
    a.out = m.out;
    a.out_ld = m.out_ld;
    a.out_f32 = m.out_f32;
    int MR = 1;
    int rc0 = fused_rows(m, &MR);
    if (rc0) return rc0;
    const int kbf = MR <= 4 ? 8 : 4;
    fused_fn fn = pick_fused(m, MR, false);
    if (!fn) return fail(EXL3_ERR_UNSUPPORTED, "exl3_moe_forward: fused layer for K %d / %d not built", m.Kg, m.Kd);
    // items <= sum over active experts of ceil(rows / MR) <= (pairs + active * (MR - 1)) / MR
    const int active = a.np < a.E ? a.np : a.E;
    int mi = (a.np + active * (MR - 1)) / MR;
    a.max_items = mi < a.np ? mi : a.np;
    const int nbI = a.I / 128, nbH = a.H / 128;
    // gate|up jobs: at most one per workgroup the device holds at once (EXL3MI_FUSED_JOBS overrides); the grid adds one
    // item's worth of workgroups for the last item's down jobs. Down jobs split I only as far as the staged blocks
    // need: an unsplit down job writes its rows directly, with no partial-sum round trip.
    int resident = 0;
    int rc = resident_blocks(reinterpret_cast<const void*>(fn), 256, &resident);
    if (rc) return rc;
    const int target = env_int("EXL3MI_FUSED_JOBS", resident);
    // gate|up jobs of at least kFusedMinJobRows tile-rows: more, shorter jobs add partial sums to every epilogue and,
    // past the resident grid, queue behind each other
    const int by_rows = a.H / 16 / kFusedMinJobRows > 1 ? a.H / 16 / kFusedMinJobRows : 1;
    const int by_grid = target / (a.max_items * nbI);
    a.P_gu = fused_splits(env_int("EXL3MI_FUSED_PGU", by_grid < by_rows ? by_grid : by_rows), a.H / 16, kbf);
    a.GU = nbI * a.P_gu;
    a.P_d = fused_splits(1, a.I / 16, kbf);
    a.DN = nbH * a.P_d;
    // unsplit down jobs compute their whole input from the partials (each column block of I is then rebuilt by the
    // item's nbH down jobs instead of once by a gate|up epilogue, saving that stage's round trips); with many
    // gate|up splits the partial loads cost more than the stage saves, and once the gate|up jobs fill more than half
    // of the device the rebuilt inputs' ALU work costs more than the round trip (C3 at 4 tokens: 37.5 against 38.2 us
    // with the epilogue stage; 1 and 2 tokens 0.3 - 0.5 us faster without it)
    const int64_t jgu = (int64_t)a.max_items * a.GU, grid = jgu + a.GU;
    a.direct = a.P_d == 1 && a.P_gu <= 8 && nbH <= 64 && 2 * jgu <= resident &&
               env_int("EXL3MI_FUSED_EPILOGUE", 0) == 0;
    if (a.direct) {                                      // the direct-mode instantiation (it must hold as many)
        fused_fn fd = pick_fused(m, MR, true);
        int resident_d = 0;
        if (fd && (rc = resident_blocks(reinterpret_cast<const void*>(fd), 256, &resident_d))) return rc;
        if (fd && 2 * jgu <= resident_d) fn = fd;
        else a.direct = 0;
    }
    EXL3_CHECK_ARG(grid < 0x7FFFFFFF, "exl3_moe_forward: grid too large");
    a.J_gu = (int)jgu;

    const size_t mx = a.max_items, np = a.np;
    const size_t pd = a.P_d > 1 ? mx * nbH * a.P_d * MR * 128 : 1;
    const size_t bytes = carve_size(mx * MR * a.I, 4) + carve_size(np * a.H, 4) +
                         carve_size(mx * nbI * a.P_gu * 2 * MR * 128, 4) + carve_size(pd, 4);
    const size_t n_cnt = (mx * nbI + mx * nbH + (size_t)a.M * nbH + mx) * kCS;
    Workspace ws;
    rc = workspace(bytes, n_cnt, st, &ws);
    if (rc) return rc;
    Carve c{ws.scratch, ws.scratch_bytes};
    a.abuf = c.take<float>(mx * MR * a.I);
    a.y = c.take<float>(np * a.H);
    a.part_gu = c.take<float>(mx * nbI * a.P_gu * 2 * MR * 128);
    a.part_d = c.take<float>(pd);
    if (!a.part_d) return fail(EXL3_ERR_INVALID, "moe: workspace carve failed");
    int* cn = ws.counters;
    a.cnt_gu = cn;
    a.cnt_d = a.cnt_gu + mx * nbI * kCS;
    a.cnt_tok = a.cnt_d + mx * nbH * kCS;
    a.cnt_item = a.cnt_tok + (size_t)a.M * nbH * kCS;
    a.status = ws.status;
    a.spin_max = spin_limit();
    EXL3_LAUNCH("moe_fused", fn, dim3((unsigned)grid), dim3(256), 0, st, a);
    return EXL3_OK;
}

}  // namespace exl3
