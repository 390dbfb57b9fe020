// The kernels of fkv_attn_q1.hip with the extensions (per-head-scaled fp8
// keys, top-K spike tokens) compiled in: a translation unit of their own so
// that both groups build in parallel with the same scheduling flags.
#include "fkv_attn_kernel.h"

namespace fkv {

AttnKernel attn_kernel_one_quad_ext(int D, int fmt) {
    if (D == 128) return fmt == 2 ? attn_kernel<128, 1, 2, true> : attn_kernel<128, 1, 0, true>;
    return fmt == 2 ? attn_kernel<64, 1, 2, true> : attn_kernel<64, 1, 0, true>;
}

}  // namespace fkv
