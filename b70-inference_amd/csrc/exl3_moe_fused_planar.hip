// Fused small-batch MoE layer, instantiations that read weights in PLANAR4 word order (the reference's expert blobs
// at K = 3, 5, 6, 7, where that order differs from tile order; glm/xpu/exl3xpu/moe_offload.py:68-78,
// glm/xpu/pack_store.py:35-54), in a translation unit of their own so that they compile in parallel with the others.
#include "exl3_moe_fused.h"

namespace exl3 {

template <int K>
static fused_fn pick_planar_mr(int MR) {
    return MR == 1 ? moe_fused_kernel<K, K, 1, true> : MR == 2 ? moe_fused_kernel<K, K, 2, true>
         : MR == 4 ? moe_fused_kernel<K, K, 4, true> : moe_fused_kernel<K, K, 8, true>;
}

fused_fn pick_fused_planar(int K, int MR) {
    switch (K) {
        case 3: return pick_planar_mr<3>(MR);
        case 5: return pick_planar_mr<5>(MR);
        case 6: return pick_planar_mr<6>(MR);
        case 7: return pick_planar_mr<7>(MR);
        default: return nullptr;
    }
}

}  // namespace exl3
