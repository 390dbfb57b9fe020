// The kernels of fkv_attn_qn.hip with the extensions (per-head-scaled fp8
// keys, top-K spike tokens) compiled in: a translation unit of their own so
// that both groups build in parallel with the same scheduling flags.
#include "fkv_attn_kernel.h"

namespace fkv {

namespace {

template <int D, int FMT>
AttnKernel pick_ext(int nq) {
    switch (nq) {
        case 2: return attn_kernel<D, 2, FMT, true>;
        case 3: return attn_kernel<D, 3, FMT, true>;
        default: return attn_kernel<D, 4, FMT, true>;
    }
}

}  // namespace

AttnKernel attn_kernel_quads_ext(int D, int fmt, int nq) {
    if (D == 128) return fmt == 2 ? pick_ext<128, 2>(nq) : pick_ext<128, 0>(nq);
    return fmt == 2 ? pick_ext<64, 2>(nq) : pick_ext<64, 0>(nq);
}

}  // namespace fkv
