// The kernels of fkv_attn_q1.hip with the extensions compiled in, in two
// variants: per-head-scaled fp8 keys only, and top-K spike tokens (the far
// tiles' maxima stored, scaled keys optional).  A translation unit of
// their own so that both groups build in parallel with the same scheduling
// flags.
#include "fkv_attn_kernel.h"

namespace fkv {

namespace {

template <int D, bool SPK>
AttnKernel pick_one(int fmt) {
    return fmt == 2 ? attn_kernel<D, 1, 2, true, SPK> : attn_kernel<D, 1, 0, true, SPK>;
}

}  // namespace

AttnKernel attn_kernel_one_quad_ext(int D, int fmt, bool spk) {
    if (D == 128) return spk ? pick_one<128, true>(fmt) : pick_one<128, false>(fmt);
    return spk ? pick_one<64, true>(fmt) : pick_one<64, false>(fmt);
}

}  // namespace fkv
