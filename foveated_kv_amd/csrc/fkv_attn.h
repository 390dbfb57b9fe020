// Internal declarations of the attention handle (not part of the C ABI).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/fkv.h"
#include "fkv_common.h"

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
//   kscale     : [B*Hkv] fp32 per-head fp8 key scale (1 unless set with
//                fkv_attn_set_k_scale; the kernel multiplies far scores by it)
// A TurboQuant blob (fmt 1) keeps the near tiers and near_valid and stores
// the far tier as TurboQuant records instead (layout below).
struct BlobLayout {
    int B, Hkv, D, Na, F, Na_pad, F_pad;
    int fmt;  // 0: fp8-E4M3 K / INT4 V far records, 1: TurboQuant, 2: fp8 K / group-32 INT4 V
    size_t near_k, near_v, far, far_rec, near_valid, kscale, total;
};

BlobLayout make_layout(int B, int Hkv, int D, int Na, int F, int fmt = 0);

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
// TurboQuant far record (fmt 1), one per (batch, kv head, 64-token tile):
//   [ KP: 3 bit planes x 64 tokens x D/8 bytes -- plane 0 = high bit of
//         the 2-bit Lloyd-Max index, 1 = low bit, 2 = QJL sign; lane l =
//         token l; dword k of a token: dims 32k+2i, 32k+2i+1 at bits
//         15-i, 31-i
//   | VP: per 64-dim half dh one 1 KB chunk, lane l = dim 64dh + l, four
//         dwords [high bit own, high bit other, low bit own, low bit other]
//         of the 2-bit value codes; "own" = the 32 tokens 32*(l/32).. of
//         the lane's half, "other" = the other 32; tokens 2i, 2i+1 of a
//         half at bits 15-i, 31-i
//   | SC: fp16 value-group scales as the P.V lanes read them: token t =
//         4 blk + e of the tile, group g = 2 dh + half at
//         ((2 blk + half) * 4 + e) * D/64 + dh (tq_sc_index), so a lane
//         (block blk, half) reads its tokens' scales in its own groups as
//         one 16-byte (D = 64: 8-byte) load
//   | NG: [token] u32 = fp16 key norm | fp16 residual norm << 16 ]
// Every plane bit is stored complemented (set = -1), so that
// (w & 0x80008000) | 0x3C003C00 is the pair of +-1 fp16 operands.
__host__ __device__ constexpr int64_t tq_vp_section(int D) { return (int64_t)24 * D; }
__host__ __device__ constexpr int64_t tq_sc_section(int D) { return (int64_t)40 * D; }
__host__ __device__ constexpr int64_t tq_ng_section(int D) { return (int64_t)44 * D; }
__host__ __device__ constexpr int64_t tq_record_bytes(int D) { return (int64_t)44 * D + 256; }
// fp16 index in the SC section of the scale of token 4 blk + e, group 2 dh + half
__host__ __device__ constexpr int tq_sc_index(int D, int blk, int half, int e, int dh) {
    return ((2 * blk + half) * 4 + e) * (D / 64) + dh;
}

// fp8 K + group-32 INT4 V far record (fmt 2): the fmt-0 K section, then
//   | V: per 64-dim half dh two 1 KB chunks (own, other), lane l = dim
//        64dh + l, 16 bytes = the nibbles of the 32 tokens of one half of
//        the tile ("own" = tokens 32*(l/32).., "other" = the other 32) in
//        the fmt-0 dword arrangement (dword u: 4-token groups 2u and 2u+1)
//   | SZ: [token][D/32] u32 = fp16 scale | fp16 zero << 16 of each group ]
__host__ __device__ constexpr int64_t g32_sz_section(int D) { return (int64_t)96 * D; }
__host__ __device__ constexpr int64_t g32_record_bytes(int D) { return (int64_t)104 * D; }

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

// Element i of an fp16 / bf16 / fp32 array as fp16 bits (round to nearest even).
__device__ inline uint16_t load_as_f16(const void* p, int64_t i, int dtype) {
    if (dtype == FKV_F16) return ((const uint16_t*)p)[i];
    if (dtype == FKV_BF16) return f2h(bf2f(((const uint16_t*)p)[i]));
    return f2h(((const float*)p)[i]);
}

// TurboQuant constants of a handle: the 2-bit centroids written as
// alpha + beta*sh + gamma*sl + delta*sh*sl over the +-1 index bits
// (sh = +1 for codes 2, 3; sl = +1 for codes 1, 3), the value levels as
// lvh*sh + lvl*sl, and Pi and S as the A operands of the query rotation /
// sketch MFMAs (tq_rot_index).
struct TurboConsts {
    float alpha = 0.f, beta = 0.f, gamma = 0.f, delta = 0.f, lvh = 0.f, lvl = 0.f;
    uint16_t* rot = nullptr;  // 4 * D * D bytes of fp16 operands
};

// Pi (mat 0) and S (mat 1) as fp16, laid out so that lane l of a wave
// reads row i = 64 * rg + l of M, k-steps 2 * s2 and 2 * s2 + 1 (columns
// 8 * s2 .. 8 * s2 + 7), as one 16-byte load:
//   [mat][s2 < D/8][i < D][8 halves]
__host__ __device__ inline int64_t tq_rot_index(int D, int mat, int i, int j) {
    return (((int64_t)mat * (D / 8) + j / 8) * D + i) * 8 + j % 8;
}

}  // namespace fkv

struct fkv_attn_impl {
    fkv::BlobLayout L;
    uint8_t* blob = nullptr;
    float margin = 0.f;
    // Call workspace, allocated once by the handle's first call for that
    // call's query-head count and never re-allocated (a captured HIP graph
    // keeps these pointers): split partials for the largest launch plan any
    // decode length can produce, the per-row arrival counters, an fp16 copy
    // of bf16 / f32 queries.
    int ws_hq = 0;          // query heads the workspace is sized for (0: none yet)
    float* ws = nullptr;    // split partials
    size_t ws_floats = 0;
    uint16_t* qbuf = nullptr;
    int* arrive = nullptr;  // per-row split arrival counters (zero between calls)
    size_t arrive_n = 0;
    int near_plan = 0;      // expected near tiles per row: max near_valid / 64, rounded up
    int device = 0;
    int target_wgs = 256;   // workgroups a launch aims for (FKV_TARGET_WGS at creation)
    bool fused_merge = true;  // in-kernel split merge (FKV_FUSED_MERGE at creation)
    // XCD count of the device's workgroup -> XCD dispatch rule (xcd_rule);
    // 0: rule not confirmed or FKV_XCD_LOCAL=0 at creation (merge through
    // memory)
    int xcd_mod = 0;
    fkv::TurboConsts tq;    // fmt 1 only
    // Top-K spikes (fkv_attn_set_spike_k): tokens per query head, and the
    // selection's buffers for spk_hq query heads (allocated with the
    // workspace, or by the setter after it): far tile maxima, thresholds,
    // the attention kernel's own flag / argmax
    int spike_k = 1;
    bool has_kscale = false;  // fkv_attn_set_k_scale was called (else the scales are 1)
    int spk_hq = 0;
    float* spk_tmax = nullptr;
    float* spk_thr = nullptr;
    int32_t* spk_flags = nullptr;
    int32_t* spk_tokens = nullptr;
    int* spk_cand_n = nullptr;   // per head: candidates found (zero between calls)
    int* spk_arrive = nullptr;   // per (batch, KV head, head quad): workgroups done (zero between calls)
    float* spk_cand_s = nullptr; // per head: up to 64 * FKV_MAX_SPIKE_K candidate scores
    int* spk_cand_t = nullptr;   // ... and their tokens
    // Every call reuses the workspace and the selection's buffers, so a call
    // on another stream than the handle's last eager call first waits for
    // that call's work (an event recorded after each eager call's launches;
    // calls under graph capture neither wait nor record: a captured graph's
    // replays are ordered by whoever launches them)
    hipEvent_t order_ev = nullptr;
    hipStream_t order_st = nullptr;
    bool order_pending = false;
};

struct fkv_attn : fkv_attn_impl {};

namespace fkv {

int grid_for(int64_t n, int block);

// How one call is launched: query heads per workgroup row, rows, splits,
// and the split-partial floats it needs.
struct LaunchPlan {
    int hpg, head_groups, ng_max, rows, splits;
    int waves;      // waves per workgroup
    int wave_recs;  // split records per split (waves: one per wave, 1: merged in LDS)
    size_t ws_floats;
};
LaunchPlan plan_launch(const BlobLayout& L, int Hq, int n_decode, int target_wgs);
// The workspace a handle's first call allocates for Hq query heads: enough
// for every launch plan of that head count (any decode length).
size_t workspace_floats(const BlobLayout& L, int Hq);
int workspace_rows(const BlobLayout& L, int Hq);
// Handle construction shared by the fp8 and TurboQuant formats: allocates
// the blob (zeroed), packs the near tiers and near_valid (stream-ordered).
int attn_begin(fkv_attn_impl* h, int B, int Hkv, int D, int Na, int F, int fmt, const void* near_k,
               const void* near_v, int near_dtype, const int32_t* near_valid, float margin, hipStream_t st);
// Synchronous end of construction: reads near_valid back for the split plan.
int attn_finish(fkv_attn_impl* h, hipStream_t st);

}  // namespace fkv
