// fp8 and group-32 attention kernels of rows of one head quad (C2, C3, and
// C1's rows of 4 heads).  A translation unit of their own so that the
// Makefile can compile them with the max-ilp instruction scheduling, which
// measured fastest for them (C1 6.75 -> 6.38 us, C3 -0.05 to -0.2 us, C2
// within noise; the same strategy slowed the TurboQuant kernels down).
// Their extension-carrying twins (per-head key scales, top-K spikes) are
// in fkv_attn_q1x.hip.
#include "fkv_attn_kernel.h"

namespace fkv {

AttnKernel attn_kernel_one_quad_ext(int D, int fmt, bool spk);

AttnKernel attn_kernel_one_quad(int D, int fmt, bool ext, bool spk) {
    if (ext) return attn_kernel_one_quad_ext(D, fmt, spk);
    if (D == 128) return fmt == 2 ? attn_kernel<128, 1, 2> : attn_kernel<128, 1, 0>;
    return fmt == 2 ? attn_kernel<64, 1, 2> : attn_kernel<64, 1, 0>;
}

}  // namespace fkv
