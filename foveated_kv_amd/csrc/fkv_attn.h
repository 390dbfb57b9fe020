// Internal declarations of the attention handle (not part of the C ABI).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/fkv.h"

namespace fkv {

// Device blob of one layer.  Offsets are bytes from the blob base.  Near
// tiers are stored per (batch, kv head) in 64-token tiles arranged as the
// operands of v_mfma_f32_4x4x4f16 (16 blocks of 4 tokens); within a tile
// every lane's operand bytes are split into 16-byte chunks, chunk-major, so
// one wave load is a contiguous 1 KB:
//   near_k : lane l = token l of the tile; chunk c = dims 8c..8c+7 (fp16)
//   near_v : lane l = dim 64*dh + l; per 4-token group s (0..15) one
//            8-byte fp16 unit
// The far tier is one contiguous record per (batch, kv head, 64-token tile)
// so a wave streams a single 12.25 KB (D=128) block per tile:
//   [ K: 64*D bytes, lane l = token l, chunk c = E4M3 codes of dims
//        16c..16c+15
//   | V: 32*D bytes of INT4 nibbles, lane l = dim 64*dh + l
//   | SZ: 64 x u32 = fp16 scale | fp16 zero << 16 per token ]
//   near_valid : [Hkv] u32
struct BlobLayout {
    int B, Hkv, D, Na, F, Na_pad, F_pad;
    size_t near_k, near_v, far, far_rec, near_valid, total;
};

BlobLayout make_layout(int B, int Hkv, int D, int Na, int F);

// Far records are stored tile-major across (batch, kv head) rows: record
// (bkv, tile) sits at index tile * B*Hkv + bkv, so workgroups of different
// rows that advance through their tiles together read one compact window.
__host__ __device__ inline int64_t far_rec_index(const BlobLayout& L, int64_t bkv, int tile) {
    return (int64_t)tile * L.B * L.Hkv + bkv;
}

// Element positions inside one (batch, kv head) region of a near tier, in
// halves.
__host__ __device__ inline int64_t near_k_index(int t, int d, int D) {
    return (int64_t)(t >> 6) * 64 * D + (int64_t)(d >> 3) * 512 + (t & 63) * 8 + (d & 7);
}
__host__ __device__ inline int64_t near_v_index(int t, int d, int D) {
    const int x = (d >> 6) * 16 + ((t & 63) >> 2);  // 8-byte unit of the lane
    return (int64_t)(t >> 6) * 64 * D + (int64_t)(x >> 1) * 512 + (d & 63) * 8 + (x & 1) * 4 + (t & 3);
}
// Far record parts: byte offsets of the V and SZ sections, record size.
__host__ __device__ constexpr int64_t far_v_section(int D) { return (int64_t)64 * D; }
__host__ __device__ constexpr int64_t far_sz_section(int D) { return (int64_t)96 * D; }
__host__ __device__ constexpr int64_t far_record_bytes(int D) { return (int64_t)96 * D + 256; }
// Byte of the E4M3 code of (token t, dim d) inside its tile's K section.
__host__ __device__ inline int64_t far_k_index(int t, int d) {
    return (int64_t)(d >> 4) * 1024 + (t & 63) * 16 + (d & 15);
}
// Far V nibble of (token t, dim d) inside its tile's V section: dword index
// and bit position.  Dword u of a lane holds 4-token groups 2(u%8) (bits
// 0-7, 16-23) and 2(u%8)+1 (bits 8-15, 24-31) of dim half u/8; token e of a
// group sits at bit 16(e&1) + 4(e>>1) of its byte pair.
__host__ __device__ inline void far_v_pos(int t, int d, int64_t& dword, int& bit) {
    const int sp = (t & 63) >> 2, e = t & 3;
    const int u = (d >> 6) * 8 + (sp >> 1);
    dword = (int64_t)(u >> 2) * 256 + (d & 63) * 4 + (u & 3);
    bit = (sp & 1) * 8 + (e & 1) * 16 + (e >> 1) * 4;
}

}  // namespace fkv
