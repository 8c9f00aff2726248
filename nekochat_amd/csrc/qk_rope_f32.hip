// q/k RMSNorm + NeoX RoPE kernels instantiated for f32 activations (one translation unit per type
// keeps the build parallel).
#include "qk_rope_kernels.h"

namespace neko_hip {

QkKernel pick_qk_f32(int L, int V, int nh, bool kv, int* split) {
    return kv ? pick_lv<float, true>(L, V, nh, split) : pick_lv<float, false>(L, V, nh, split);
}

}  // namespace neko_hip
