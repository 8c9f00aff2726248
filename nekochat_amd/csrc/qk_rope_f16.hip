// q/k RMSNorm + NeoX RoPE kernels instantiated for f16 activations (one translation unit per type
// keeps the build parallel).
#include "qk_rope_kernels.h"

namespace neko_hip {

QkKernel pick_qk_f16(int L, int V, int nh, bool kv, int* split) {
    return kv ? pick_lv<half_t, true>(L, V, nh, split) : pick_lv<half_t, false>(L, V, nh, split);
}

}  // namespace neko_hip
