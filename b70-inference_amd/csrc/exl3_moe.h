// Argument blocks of the grouped MoE kernels (device pointers into the caller's tensors and the workspace).
#pragma once

#include <stdint.h>

namespace exl3 {

constexpr int kMoeMaxExperts = 3072;   // expert tables per layer (routed + shared); the align kernel keeps 4 ints each in LDS

struct RouteArgs {
    const int32_t* ids;
    const float* tw;
    int M, topk, slots, E, shared, MR;
    int* counts;                       // optional [E]
    int* n_items;                      // optional: items of <= MR rows
    int* item_e;
    int* item_p0;
    int* item_cnt;
    int* pair_tok;
    float* pair_w;
    int* pair_of;
};

struct MoeArgs {
    const uint16_t* x;
    int64_t x_ld;
    int M, H, I, topk, slots, E;
    const int32_t* ids;
    const float* tw;
    const int64_t* tables;             // [9][E]
    const int64_t* kmaps;              // [6][E] or null
    int Kg, Kd;                        // gate/up K, down K (0 = per-tile)
    int act;
    float limit;
    int shared;
    int MR, max_items;
    // routing (workspace)
    int* n_items;
    int* item_e;
    int* item_p0;
    int* item_cnt;
    int* pair_tok;
    float* pair_w;
    int* pair_of;
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
