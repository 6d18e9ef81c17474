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
    for (int j = 0; j < a.slots; ++j) {
        const int pr = a.pair_of[t * a.slots + j];
        if (pr < 0) continue;
        const float* y = a.y + (size_t)pr * a.H;
        v0 += splitk_load(y + c0);
        v1 += splitk_load(y + c1);
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

}  // namespace exl3
