// Internal declarations of the attention handle (not part of the C ABI).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/fkv.h"

namespace fkv {

// Device blob of one layer.  Offsets are bytes from the blob base; each
// tier is stored per (batch, kv head) in 64-token tiles arranged as the
// operands of v_mfma_f32_4x4x4f16 (16 blocks of 4 tokens).  Within a tile
// every lane's operand bytes are split into 16-byte chunks, chunk-major, so
// one wave load is a contiguous 1 KB.
//   near_k / far_k : lane l = token l of the tile; chunk c = dims 8c..8c+7
//                    (fp16) or 16c..16c+15 (E4M3 codes)
//   near_v / far_v : lane l = dim 64*dh + l; per 4-token group s (0..15)
//                    one 8-byte fp16 unit (near) or 16 bits of nibbles (far)
//   far_sz         : [F_pad] u32 = fp16 scale | fp16 zero << 16
//   near_valid     : [Hkv] u32
struct BlobLayout {
    int B, Hkv, D, Na, F, Na_pad, F_pad;
    size_t near_k, near_v, far_k, far_v, far_sz, near_valid, total;
};

BlobLayout make_layout(int B, int Hkv, int D, int Na, int F);

// Element positions inside one (batch, kv head) region of a tier.
// near K / near V: index in halves; far K: index in bytes.
__host__ __device__ inline int64_t near_k_index(int t, int d, int D) {
    return (int64_t)(t >> 6) * 64 * D + (int64_t)(d >> 3) * 512 + (t & 63) * 8 + (d & 7);
}
__host__ __device__ inline int64_t near_v_index(int t, int d, int D) {
    const int x = (d >> 6) * 16 + ((t & 63) >> 2);  // 8-byte unit of the lane
    return (int64_t)(t >> 6) * 64 * D + (int64_t)(x >> 1) * 512 + (d & 63) * 8 + (x & 1) * 4 + (t & 3);
}
__host__ __device__ inline int64_t far_k_index(int t, int d, int D) {
    return (int64_t)(t >> 6) * 64 * D + (int64_t)(d >> 4) * 1024 + (t & 63) * 16 + (d & 15);
}
// Far V nibble of (token t, dim d): dword index and bit position.  Dword u
// of a lane holds 4-token groups 2(u%8) (bits 0-7, 16-23) and 2(u%8)+1
// (bits 8-15, 24-31) of dim half u/8; token e of a group sits at bit
// 16(e&1) + 4(e>>1) of its byte pair.
__host__ __device__ inline void far_v_pos(int t, int d, int D, int64_t& dword, int& bit) {
    const int sp = (t & 63) >> 2, e = t & 3;
    const int u = (d >> 6) * 8 + (sp >> 1);
    dword = (int64_t)(t >> 6) * 8 * D + (int64_t)(u >> 2) * 256 + (d & 63) * 4 + (u & 3);
    bit = (sp & 1) * 8 + (e & 1) * 16 + (e >> 1) * 4;
}

}  // namespace fkv
