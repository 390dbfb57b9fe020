// The kernels of fkv_attn_qn.hip with the extensions compiled in, in two
// variants: per-head-scaled fp8 keys only, and top-K spike tokens (the far
// tiles' maxima stored, scaled keys optional).  A translation unit of
// their own so that both groups build in parallel with the same scheduling
// flags.
#include "fkv_attn_kernel.h"

namespace fkv {

namespace {

template <int D, int FMT, bool SPK>
AttnKernel pick_ext(int nq) {
    switch (nq) {
        case 2: return attn_kernel<D, 2, FMT, true, SPK>;
        case 3: return attn_kernel<D, 3, FMT, true, SPK>;
        default: return attn_kernel<D, 4, FMT, true, SPK>;
    }
}

template <int D, bool SPK>
AttnKernel pick_fmt(int fmt, int nq) {
    return fmt == 2 ? pick_ext<D, 2, SPK>(nq) : pick_ext<D, 0, SPK>(nq);
}

}  // namespace

AttnKernel attn_kernel_quads_ext(int D, int fmt, int nq, bool spk) {
    if (D == 128) return spk ? pick_fmt<128, true>(fmt, nq) : pick_fmt<128, false>(fmt, nq);
    return spk ? pick_fmt<64, true>(fmt, nq) : pick_fmt<64, false>(fmt, nq);
}

}  // namespace fkv
