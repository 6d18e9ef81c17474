// Argument blocks of the grouped MoE kernels (device pointers into the caller's tensors and the workspace).
#pragma once

#include <stdint.h>

namespace exl3 {

constexpr int kMoeMaxExperts = 2048;   // expert tables per layer (routed + shared); the align kernel keeps 5 ints each in LDS
constexpr int kMoeSmallRows = 8;       // experts with at most this many rows in a call take the GEMV kernels
constexpr int kMfmaRows = 64;          // row block of the MFMA grouped GEMM

// Row class of an MFMA block (0: <= 16 rows, 1: <= 32, 2: <= 64): each class runs its own kernel instance sized for
// its row groups, so that small blocks get the register budget (and occupancy) of a small block.
__host__ __device__ constexpr int mfma_row_class(int cnt) { return cnt <= 16 ? 0 : cnt <= 32 ? 1 : 2; }

// One work unit of the GEMV kernels: up to 8 rows (pairs) of one expert, with everything a workgroup needs so that a
// single uniform load replaces the table lookups. Items past the last real one have cnt == 0.
struct alignas(256) ItemDesc {
    int32_t e, p0, cnt, pad;
    int32_t tok[8];                    // token of each row
    float w[8];                        // routing weight of each row (1 for the shared expert)
    int64_t tab[9];                    // the expert's (trellis, suh, svh) addresses for gate, up, down
    int64_t km[6];                     // (kmap, woff) addresses for gate, up, down when K is per tile
};
static_assert(sizeof(ItemDesc) == 256, "item descriptor layout");

struct RouteArgs {
    const int32_t* ids;
    const float* tw;
    int M, topk, slots, E, shared, MR;
    int* counts;                       // optional [E]
    int* n_items;                      // optional: items of <= MR rows
    ItemDesc* items;                   // optional [max_items]
    int max_items;
    const int64_t* tables;             // [9][E] (read when items are built)
    const int64_t* kmaps;              // [6][E] or null
    int use_mfma, MB;                  // experts with more than MR rows -> blocks of MB rows for the MFMA kernels
    ItemDesc* blocks;                  // [max_blocks]
    int max_blocks;
    int* cls_list;                     // optional [3][max_blocks]: block indices by row class (<= 16, 32, 64 rows)
    int* cls_cnt;                      // [3]
    int* pair_tok;
    float* pair_w;
    int* pair_of;
    int* pair_e;                       // optional [M * slots]: expert of each pair in sorted order, -1 past the valid
                                       // pairs
    int* tok_nvalid;                   // optional [M]: valid slots per token; tokens with none get a zero output row
    void* out;
    int64_t out_ld;
    int out_f32, H;
    int held;                          // align_kernel: each thread holds its (at most 8) pairs in registers and
                                       // counts the tokens' valid slots in LDS (M more ints of dynamic LDS)
    int staged;                        // align_kernel (held): the sorted pair arrays are built in LDS (3 * M * slots
                                       // more ints) and written out with coalesced stores
};

constexpr int kFusedRouteMaxE = 512;    // logits per row that the fused layer's in-layer routing handles (8 per lane)
constexpr int kFusedRouteMaxRows = 4;   // tokens up to which the routed entry point ranks inside the fused layer

struct MoeArgs {
    const uint16_t* x;
    int64_t x_ld;
    int M, H, I, topk, slots, E;
    const int32_t* ids;
    const float* tw;
    const int64_t* tables;             // [9][E]
    const int64_t* kmaps;              // [6][E] or null
    int uniform;                       // tables[i][e] == tb[i] + e * ts[i] for every entry (host-known layout)
    int64_t tb[9], ts[9];
    int Kg, Kd;                        // gate/up K, down K (0 = per-tile)
    int gu_tn;                         // tiles per tile-row of the gate and up trellises (uniform K): I / 16, or
                                       // 2 I / 16 for the reference's expert blob (gate and up tiles of a tile-row
                                       // side by side, up at gate + I / 16 tiles)
    int planar;                        // weights in PLANAR4 word order (the reference's blobs at K = 3, 5, 6, 7):
                                       // picks the kernels' PL instantiations (host side only)
    // routing from logits inside the fused layer (null: ids / tw hold the routing): softmax over logits (+ rbias)
    // -> top-k -> renormalised, picks written to ids_out / tw_out
    const float* logits;
    int64_t lg_ld;
    int n_logits;
    const float* rbias;
    int32_t* ids_out;
    float* tw_out;
    int act;
    float limit;
    int shared;
    int MR, max_items;
    // routing (workspace)
    int* n_items;
    const ItemDesc* items;
    const ItemDesc* blocks;            // MFMA row blocks (cnt == 0 past the last)
    int max_blocks;
    const int* cls_list;               // [3][max_blocks] block indices by row class (<= 16, <= 32, <= 64 rows)
    const int* cls_cnt;                // [3] blocks per class
    _Float16* xh;                      // [pairs][2][H] transformed gate / up inputs of MFMA rows
    float* xsum;                       // [pairs][2][H / 128] block sums of xh (the MFMA rows' affine term)
    float* asum;                       // [pairs][I / 128] block sums of abuf (MFMA rows)
    int* pair_tok;
    float* pair_w;
    int* pair_of;
    int* pair_e;                       // [pairs] expert of each pair in sorted order, -1 past the valid pairs (MFMA
                                       // path)
    int* tok_nvalid;                   // [M] valid slots per token
    int* cnt_tok;                      // [M][H/128] combine arrival counters
    // intermediates (workspace)
    uint16_t* abuf;                    // [pairs][I] fp16, Hadamard-domain down input
    float* y;                          // [pairs][H] fp32, weighted expert outputs
    float* part_gu;
    int* cnt_gu;
    int P_gu, nblk_h;
    float* part_d;
    int* cnt_d;
    int P_d, nblk_i;
    // output
    void* out;
    int64_t out_ld;
    int out_f32;
};

}  // namespace exl3
