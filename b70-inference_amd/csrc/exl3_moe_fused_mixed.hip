// Fused small-batch MoE layer, instantiations whose gate/up bitrate differs from the down bitrate (one translation
// unit of its own so that it compiles in parallel with the equal-bitrate ones): down one or two bits above gate/up,
// the usual way a mixed-bitrate quant spends its bits (C4: gate/up K=2, down K=3; per-projection K as in
// dsv41/xpu/csrc/dsv_moe.sycl:157-170).
#include "exl3_moe_fused.h"

namespace exl3 {

template <int KG, int KD, bool D>
static fused_fn pick_mixed_kd(int MR) {
    return MR == 1 ? moe_fused_kernel<KG, KD, 1, false, D> : MR == 2 ? moe_fused_kernel<KG, KD, 2, false, D>
         : MR == 4 ? moe_fused_kernel<KG, KD, 4, false, D> : moe_fused_kernel<KG, KD, 8, false, D>;
}

template <int KG>
static fused_fn pick_mixed_mr(int Kd, int MR, bool direct) {
    constexpr int K1 = KG + 1 <= 8 ? KG + 1 : 8, K2 = KG + 2 <= 8 ? KG + 2 : 8;
    if (Kd == KG + 1 && KG + 1 <= 8)
        return direct ? pick_mixed_kd<KG, K1, true>(MR) : pick_mixed_kd<KG, K1, false>(MR);
    if (Kd == KG + 2 && KG + 2 <= 8)
        return direct ? pick_mixed_kd<KG, K2, true>(MR) : pick_mixed_kd<KG, K2, false>(MR);
    return nullptr;
}

fused_fn pick_fused_mixed(int Kg, int Kd, int MR, bool direct) {
    switch (Kg) {
        case 1: return pick_mixed_mr<1>(Kd, MR, direct);
        case 2: return pick_mixed_mr<2>(Kd, MR, direct);
        case 3: return pick_mixed_mr<3>(Kd, MR, direct);
        case 4: return pick_mixed_mr<4>(Kd, MR, direct);
        case 5: return pick_mixed_mr<5>(Kd, MR, direct);
        case 6: return pick_mixed_mr<6>(Kd, MR, direct);
        case 7: return pick_mixed_mr<7>(Kd, MR, direct);
        default: return nullptr;
    }
}

}  // namespace exl3
