// Fused small-batch MoE layer, instantiations that read weights in PLANAR4 word order (the reference's expert blobs
// at K = 3, 5, 6, 7, where that order differs from tile order; glm/xpu/exl3xpu/moe_offload.py:68-78,
// glm/xpu/pack_store.py:35-54), in a translation unit of their own so that they compile in parallel with the others.
#include "exl3_moe_fused.h"

namespace exl3 {

template <int K, bool D>
static fused_fn pick_planar_mr(int MR) {
    return MR == 1 ? moe_fused_kernel<K, K, 1, true, D> : MR == 2 ? moe_fused_kernel<K, K, 2, true, D>
         : MR == 4 ? moe_fused_kernel<K, K, 4, true, D> : moe_fused_kernel<K, K, 8, true, D>;
}

fused_fn pick_fused_planar(int K, int MR, bool direct) {
    switch (K) {
        case 3: return direct ? pick_planar_mr<3, true>(MR) : pick_planar_mr<3, false>(MR);
        case 5: return direct ? pick_planar_mr<5, true>(MR) : pick_planar_mr<5, false>(MR);
        case 6: return direct ? pick_planar_mr<6, true>(MR) : pick_planar_mr<6, false>(MR);
        case 7: return direct ? pick_planar_mr<7, true>(MR) : pick_planar_mr<7, false>(MR);
        default: return nullptr;
    }
}

}  // namespace exl3
