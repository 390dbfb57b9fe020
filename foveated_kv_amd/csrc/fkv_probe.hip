// HBM streaming-read probe: the practical read-bandwidth ceiling of the
// device, measured with the same 16-byte-per-lane, 1-KB-per-wave access
// pattern the attention kernel uses.  Benchmark utility only.
#include <hip/hip_runtime.h>

#include <string>

#include "fkv_common.h"
#include "../../include/fkv.h"

namespace fkv {

typedef uint32_t probe_u4 __attribute__((ext_vector_type(4)));

// Grid-stride read of n 16-byte words, U loads in flight per lane per
// iteration; the words are folded with XOR so the loads cannot be elided.
template <int U, bool NT>
__global__ __launch_bounds__(256) void read_probe_kernel(const probe_u4* __restrict__ p, int64_t n,
                                                         uint32_t* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (U - 1) * stride < n; i += U * stride) {
        probe_u4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = NT ? __builtin_nontemporal_load(p + i + u * stride) : p[i + u * stride];
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n; i += stride) {
        const probe_u4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc ^= __shfl_xor(acc, o, kWave);
    if (threadIdx.x % kWave == 0) out[blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave] = acc;
}

}  // namespace fkv

extern "C" int fkv_hbm_read_probe(const void* buf, int64_t bytes, int32_t unroll, int32_t nontemporal,
                                  int32_t blocks, uint32_t* out, void* stream) {
    using fkv::set_error;
    if (!buf || !out || bytes < 16 || bytes % 16 != 0)
        return set_error("fkv_hbm_read_probe: buffer must be non-NULL and a positive multiple of 16 bytes");
    if (blocks <= 0 || blocks > (1 << 20)) return set_error("fkv_hbm_read_probe: blocks must be in [1, 2^20]");
    const int64_t n = bytes / 16;
    hipStream_t st = (hipStream_t)stream;
    const fkv::probe_u4* p = (const fkv::probe_u4*)buf;
#define FKV_PROBE(U)                                                                                        \
    if (nontemporal) hipLaunchKernelGGL((fkv::read_probe_kernel<U, true>), dim3(blocks), dim3(256), 0, st, p, n, out); \
    else hipLaunchKernelGGL((fkv::read_probe_kernel<U, false>), dim3(blocks), dim3(256), 0, st, p, n, out)
    switch (unroll) {
        case 1: FKV_PROBE(1); break;
        case 2: FKV_PROBE(2); break;
        case 4: FKV_PROBE(4); break;
        case 8: FKV_PROBE(8); break;
        default: return set_error("fkv_hbm_read_probe: unroll must be 1, 2, 4 or 8");
    }
#undef FKV_PROBE
    return fkv::check_hip(hipGetLastError(), "read_probe_kernel launch");
}
