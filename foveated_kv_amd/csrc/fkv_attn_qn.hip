// fp8 and group-32 attention kernels of rows of 2-4 head quads (GQA groups
// of 5-16 query heads per KV head, e.g. C5's 8).
// A translation unit of their own so that the Makefile can compile them
// with the iterative-ilp instruction scheduling, which measured fastest for
// them (C5 29.9 -> 29.0 us).  Their extension-carrying twins (per-head key
// scales, top-K spikes) are in fkv_attn_qnx.hip.
#include "fkv_attn_kernel.h"

namespace fkv {

namespace {

template <int D, int FMT>
AttnKernel pick(int nq) {
    switch (nq) {
        case 2: return attn_kernel<D, 2, FMT>;
        case 3: return attn_kernel<D, 3, FMT>;
        default: return attn_kernel<D, 4, FMT>;
    }
}

}  // namespace

AttnKernel attn_kernel_quads_ext(int D, int fmt, int nq, bool spk);

AttnKernel attn_kernel_quads(int D, int fmt, int nq, bool ext, bool spk) {
    if (ext) return attn_kernel_quads_ext(D, fmt, nq, spk);
    if (D == 128) return fmt == 2 ? pick<128, 2>(nq) : pick<128, 0>(nq);
    return fmt == 2 ? pick<64, 2>(nq) : pick<64, 0>(nq);
}

}  // namespace fkv
