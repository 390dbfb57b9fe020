// Internal declarations of the attention handle (not part of the C ABI).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/fkv.h"

namespace fkv {

// Device blob of one layer.  Offsets are bytes from the blob base.
//   near_k   [B*Hkv][Na_pad/64][D/8][64 lanes][8 halves]   token-parallel tiles
//   near_v   [B*Hkv][Na_pad][D] fp16 rows
//   far_k    [B*Hkv][F_pad/64][D/16][64 lanes][16 codes]   token-parallel tiles
//   far_v    [B*Hkv][F_pad/GS][64 lanes][4 x u32]          d-parallel groups
//   far_sz   [B*Hkv][F_pad] u32 = fp16 scale | fp16 zero << 16
//   near_valid [Hkv] u32
struct BlobLayout {
    int B, Hkv, D, Na, F, Na_pad, F_pad;
    size_t near_k, near_v, far_k, far_v, far_sz, near_valid, total;
};

BlobLayout make_layout(int B, int Hkv, int D, int Na, int F);

}  // namespace fkv
