// Fused two-tier split-K decode attention for gfx950 (fp8-E4M3 K / INT4 V far
// tier, fp16 near tier, fp16 decode buffer) and the per-layer device blob.
//
// Replaces the reference's FoveatedHandle + foveated_2tier Metal kernel
// (csrc/foveated_attn.cpp:83-254, csrc/kernels/foveated_attn.metal:181-432).
//
// Work decomposition: one workgroup of 4 waves per (batch, kv_head, split)
// serves up to 16 query heads of the GQA group (as quads of 4), so each
// compressed byte is read from HBM once.  A wave takes 64-token tiles; both
// contractions run on the matrix cores with the 16-block
// v_mfma_f32_4x4x4f16 (fp16 operands, fp32 accumulation), so a GQA group of
// 4 heads wastes no MFMA lanes and no softmax work:
//   scores  block b = tokens 4b..4b+3:   S[t][h] += K[t][4s..4s+3] . q[h][4s..4s+3]
//   output  block b = dims 4b..4b+3:     O[h][d] += P[4g..4g+3][h] . V[4g..4g+3][d]
//           with the weights of token group g broadcast to every block
//           (cbsz = 4, abid = g).
// The score MFMA leaves each lane the 4 weights that the P.V MFMA takes as
// its A operand, so softmax weights never leave registers.
// E4M3 keys are widened to fp16 with the native converter (exact); INT4
// values are widened exactly by inserting the nibble into an fp16 mantissa
// (16 + c), weights are p*scale, and the zero point and constant offsets
// are folded into per-head scalars.  The fp16 query is used unscaled (exact
// products); 1/sqrt(D) is applied to the fp32 scores.
// The blob stores every tier pre-arranged in these operand layouts so each
// lane's operand bytes are contiguous and every wave load is a contiguous
// 1 KB.  Split partials are merged inside the kernel by the last split of a
// row to arrive (merge_kernel, a separate launch, is kept for comparison).
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

#include "fkv_attn.h"
#include "fkv_common.h"

#include "fkv_attn_kernel.h"

namespace fkv {

#ifdef FKV_PHASE_STAMPS
__device__ unsigned long long fkv_stamps[kStampSlots * kStampWGs];
#endif

// ---------------------------------------------------------------------------
// Blob layout
// ---------------------------------------------------------------------------

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

BlobLayout make_layout(int B, int Hkv, int D, int Na, int F, int fmt) {
    BlobLayout L{};
    L.fmt = fmt;
    L.B = B;
    L.Hkv = Hkv;
    L.D = D;
    L.Na = Na;
    L.F = F;
    L.Na_pad = (int)round_up(Na, kTile);
    L.F_pad = (int)round_up(F, kTile);
    const size_t bkv = (size_t)B * Hkv;
    size_t off = 0;
    auto place = [&](size_t bytes) {
        size_t p = off;
        off = align256(off + bytes);
        return p;
    };
    L.near_k = place(bkv * L.Na_pad * D * 2);
    L.near_v = place(bkv * L.Na_pad * D * 2);
    L.far_rec = (size_t)(fmt == 1 ? tq_record_bytes(D) : fmt == 2 ? g32_record_bytes(D) : far_record_bytes(D));
    L.far = place(bkv * (L.F_pad / kTile) * L.far_rec);
    L.near_valid = place((size_t)Hkv * 4);
    L.kscale = place(bkv * 4);
    L.total = off;
    return L;
}

// ---------------------------------------------------------------------------
// Blob packing kernels (handle construction; csrc/foveated_attn.cpp:83-128)
// ---------------------------------------------------------------------------

// One thread per (bkv, token, 16-dim block): near K and V into their tile
// layouts (fkv_attn.h); slots >= Na are zero.
__global__ void pack_near_kernel(const void* __restrict__ nk, const void* __restrict__ nv,
                                 int dtype, BlobLayout L, uint8_t* __restrict__ blob) {
    const int D = L.D, NB = D / 16;
    const int64_t n = (int64_t)L.B * L.Hkv * L.Na_pad * NB;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int blk = (int)(i % NB);
        const int64_t r = i / NB;
        const int t = (int)(r % L.Na_pad);
        const int64_t bkv = r / L.Na_pad;
        uint16_t* kd = (uint16_t*)(blob + L.near_k) + bkv * (int64_t)L.Na_pad * D;
        uint16_t* vd = (uint16_t*)(blob + L.near_v) + bkv * (int64_t)L.Na_pad * D;
        for (int e = 0; e < 16; e++) {
            const int d = blk * 16 + e;
            const int64_t src = (bkv * L.Na + t) * D + d;
            kd[near_k_index(t, d, D)] = t < L.Na ? load_as_f16(nk, src, dtype) : 0;
            vd[near_v_index(t, d, D)] = t < L.Na ? load_as_f16(nv, src, dtype) : 0;
        }
    }
}

// Far K codes into the tile layout; exponent-0 codes are written as signed
// zero (the reference LUT ignores their mantissa); NaN codes 0x7F/0xFF are
// reported through *bad.
__global__ void pack_far_k_kernel(const uint8_t* __restrict__ fk, BlobLayout L,
                                  uint8_t* __restrict__ blob, unsigned* __restrict__ bad) {
    const int D = L.D, NB = D / 16;
    const int64_t n = (int64_t)L.B * L.Hkv * L.F_pad * NB;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int blk = (int)(i % NB);
        const int64_t r = i / NB;
        const int t = (int)(r % L.F_pad);
        const int64_t bkv = r / L.F_pad;
        uint8_t* dst = blob + L.far + far_rec_index(L, bkv, t / kTile) * (int64_t)L.far_rec;
        for (int e = 0; e < 16; e++) {
            const int d = blk * 16 + e;
            uint8_t b = 0;
            if (t < L.F) {
                b = fk[(bkv * L.F + t) * D + d];
                if ((b & 0x7F) == 0x7F) atomicOr(bad, 1u);
                if ((b & 0x78) == 0) b &= 0x80;
            }
            dst[far_k_index(t, d)] = b;
        }
    }
}

// Far V nibbles: one thread builds one dword of the tile layout (8 nibbles:
// 2 four-token groups of one dim); thread (kg=0 lanes) also packs the
// per-token scale / zero.
__global__ void pack_far_v_kernel(const uint8_t* __restrict__ fv, const void* __restrict__ fvs,
                                  const void* __restrict__ fvz, int sz_dtype, BlobLayout L,
                                  uint8_t* __restrict__ blob) {
    const int D = L.D;
    const int64_t words_per_bkv = (int64_t)L.F_pad * D / 8;
    const int64_t n = (int64_t)L.B * L.Hkv * words_per_bkv;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t bkv = i / words_per_bkv;
        const int64_t w = i % words_per_bkv;
        // invert the dword position: tile, chunk, lane, word-in-chunk
        const int tile = (int)(w / (8 * D));
        const int rem = (int)(w % (8 * D));
        const int c = rem / 256, lane = (rem % 256) / 4, q = rem % 4;
        const int u = c * 4 + q, dh = u / 8, spair = u % 8;
        const int d = dh * 64 + lane;
        uint32_t word = 0;
        for (int bp = 0; bp < 2; bp++)
            for (int e = 0; e < 4; e++) {
                const int t = tile * 64 + (2 * spair + bp) * 4 + e;
                uint32_t code = 0;
                if (t < L.F) code = (fv[(bkv * L.F + t) * (D / 2) + d / 2] >> (4 * (d & 1))) & 15u;
                word |= code << (bp * 8 + (e & 1) * 16 + (e >> 1) * 4);
            }
        ((uint32_t*)(blob + L.far + far_rec_index(L, bkv, tile) * (int64_t)L.far_rec +
                     far_v_section(D)))[rem] = word;
    }
    const int64_t nt = (int64_t)L.B * L.Hkv * L.F_pad;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nt;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(i % L.F_pad);
        const int64_t bkv = i / L.F_pad;
        uint32_t sz = 0;
        if (t < L.F) {
            const int64_t k = bkv * L.F + t;
            sz = (uint32_t)load_as_f16(fvs, k, sz_dtype) | ((uint32_t)load_as_f16(fvz, k, sz_dtype) << 16);
        }
        ((uint32_t*)(blob + L.far + far_rec_index(L, bkv, t / kTile) * (int64_t)L.far_rec +
                     far_sz_section(D)))[t % kTile] = sz;
    }
}

// Group-32 far V (fmt 2): one thread per output dword of the V section
// (chunk c = 2*dh + half-select, lane, word u), and per token the group
// scale | zero words.
__global__ void pack_far_v_g32_kernel(const uint8_t* __restrict__ fv, const void* __restrict__ fvs,
                                      const void* __restrict__ fvz, int sz_dtype, BlobLayout L,
                                      uint8_t* __restrict__ blob) {
    const int D = L.D, NG = D / 32;
    const int64_t words_per_tile = (int64_t)8 * D;  // 32*D bytes of nibbles
    const int64_t nt = L.F_pad / kTile;
    const int64_t n = (int64_t)L.B * L.Hkv * nt * words_per_tile;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int rem = (int)(i % words_per_tile);
        const int64_t r = i / words_per_tile;
        const int tile = (int)(r % nt);
        const int64_t bkv = r / nt;
        const int c = rem / 256, lane = (rem % 256) / 4, u = rem % 4;
        const int dh = c >> 1, other = c & 1;
        const int d = dh * 64 + lane;
        const int half = lane >> 5;
        const int base = 32 * (other ? 1 - half : half);
        uint32_t word = 0;
        for (int bp = 0; bp < 2; bp++)
            for (int e = 0; e < 4; e++) {
                const int t = tile * kTile + base + (2 * u + bp) * 4 + e;
                uint32_t code = 0;
                if (t < L.F) code = (fv[(bkv * L.F + t) * (D / 2) + d / 2] >> (4 * (d & 1))) & 15u;
                word |= code << (bp * 8 + (e & 1) * 16 + (e >> 1) * 4);
            }
        ((uint32_t*)(blob + L.far + far_rec_index(L, bkv, tile) * (int64_t)L.far_rec + far_v_section(D)))[rem] = word;
    }
    const int64_t ntok = (int64_t)L.B * L.Hkv * L.F_pad;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < ntok;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(i % L.F_pad);
        const int64_t bkv = i / L.F_pad;
        uint32_t* sz = (uint32_t*)(blob + L.far + far_rec_index(L, bkv, t / kTile) * (int64_t)L.far_rec +
                                   g32_sz_section(D)) + (t % kTile) * NG;
        for (int g = 0; g < NG; g++) {
            uint32_t w = 0;
            if (t < L.F) {
                const int64_t k = (bkv * L.F + t) * NG + g;
                w = (uint32_t)load_as_f16(fvs, k, sz_dtype) | ((uint32_t)load_as_f16(fvz, k, sz_dtype) << 16);
            }
            sz[g] = w;
        }
    }
}

__global__ void pack_valid_kernel(const int32_t* __restrict__ nv, int Hkv, BlobLayout L,
                                  uint8_t* __restrict__ blob) {
    int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h < Hkv) {
        int v = nv[h];
        v = v < 0 ? 0 : (v > L.Na ? L.Na : v);
        ((uint32_t*)(blob + L.near_valid))[h] = (uint32_t)v;
    }
}

// The blob's per-head fp8 key scales: 1 (src NULL) or src[i]; a scale that
// is not a positive finite number raises *bad.
__global__ void fill_kscale_kernel(const float* __restrict__ src, int n, BlobLayout L, uint8_t* __restrict__ blob,
                                   unsigned* bad) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = src ? src[i] : 1.0f;
    if (!(v > 0.f && v <= 3.402823466e38f)) *bad = 1u;
    ((float*)(blob + L.kscale))[i] = v;
}

// E4M3 -> fp16 with the converter the fused kernel uses (4 codes per thread)
__global__ void e4m3_decode_kernel(const uint8_t* __restrict__ codes, uint16_t* __restrict__ out, int64_t n4) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t w = ((const uint32_t*)codes)[i];
        const fkv_h2 lo = e4m3x2_to_h2(w, false), hi = e4m3x2_to_h2(w, true);
        uint2 o;
        o.x = as_u32(lo);
        o.y = as_u32(hi);
        ((uint2*)out)[i] = o;
    }
}

__global__ void cast_to_f16_kernel(const void* __restrict__ src, int dtype, int64_t n,
                                   uint16_t* __restrict__ dst) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = load_as_f16(src, i, dtype);
}

// Split-K merge as its own launch (in-kernel merge switched off): one wave
// per (row, head), the same per-head merge as the in-kernel one.
template <int D>
__global__ __launch_bounds__(64) void merge_kernel(AttnArgs a) {
    constexpr int RS = kHdr + D;
    const int row = blockIdx.x, g = blockIdx.y;
    const int hgrp = row % a.head_groups;
    const int64_t bkv = row / a.head_groups;
    const int b = (int)(bkv / a.L.Hkv), kvh = (int)(bkv % a.L.Hkv);
    const int head0 = kvh * a.G + hgrp * a.hpg;
    const int ng = min(a.hpg, a.G - hgrp * a.hpg);
    if (g >= ng) return;
    const int ns = a.num_splits * a.wave_recs;
    const float* src = a.ws + (int64_t)row * ns * min(a.hpg, a.G) * RS;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, ns * ng * RS * 4, 0x00020000);
    merge_heads<D, 1, true>(a, rs, ns, ng, g, 1, (int)threadIdx.x, (int64_t)b * a.Hq + head0 + g);
}

// ---------------------------------------------------------------------------
// Top-K spike selection (spike_k > 1; the benchmark's "up to 32 far tokens
// per head per step", an extension of the reference's one token per query
// head, csrc/kernels/foveated_attn.metal:323-327, 427-430)
// ---------------------------------------------------------------------------

struct SelectArgs {
    const uint8_t* blob;
    BlobLayout L;
    const uint16_t* q;          // (B, Hq, D) fp16: the query the attention kernel read
    int Hq, G, K;
    float inv_sqrt_d;
    const float* tmax;          // (B*Hq, ntf) far tile maxima
    int ntf;
    const float* thr;           // (B*Hq) min_near + margin
    const int32_t* flags_in;    // (B*Hq) the attention kernel's flag and first-index argmax
    const int32_t* tokens_in;
    int32_t* flags;             // (B*Hq) number of spiking tokens, at most K
    int32_t* tokens;            // (B*Hq, K)
    const float* kscale;        // (B*Hkv) per-head fp8 key scales, or NULL (1)
    // candidate buffers: per head a count (zero between calls) and up to
    // cap (score, token) pairs; per (batch, KV head, head quad) the
    // workgroups that have finished (zero between calls)
    int* cand_n;                // (B*Hq)
    int* arrive;                // (B*Hkv*quads)
    float* cand_s;              // (B*Hq, cap)
    int* cand_t;                // (B*Hq, cap)
    int cap;                    // 64 * K
#ifdef FKV_PHASE_STAMPS
    unsigned long long* stamps;  // the attention kernel's stamp array; slots 32.. of each workgroup
#endif
};

// Phase stamps of the candidates kernel (the -DFKV_PHASE_STAMPS build):
// slots 32 entry, 33 tile maxima staged, 34 cuts known, 35 + w wave w done,
// 39 + w wave w's query operands loaded, 43 + w wave w's last batch begun,
// 47 the quad's selection done (its last workgroup), and of wave w's first
// batch: 48 + w begun, 52 + w rescored, 56 + w its slots reserved.
#ifdef FKV_PHASE_STAMPS
#define FKV_SEL_STAMP(cond, slot)                                                                            \
    do {                                                                                                    \
        if (cond) {                                                                                         \
            const int wg_ = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;                 \
            if (wg_ < kStampWGs) a.stamps[kStampSlots * wg_ + 32 + (slot)] = __builtin_amdgcn_s_memrealtime(); \
        }                                                                                                   \
    } while (0)
#else
#define FKV_SEL_STAMP(cond, slot) \
    do {                          \
    } while (0)
#endif

// Workgroups per (batch, KV head, head quad) of the first selection
// kernel, and the far tiles per head whose maxima a workgroup stages in
// LDS (beyond that it reads them from memory).
constexpr int kSelParts = 8;
constexpr int kSelStage = 4096;
constexpr int kSelWaves = 4;
// Far tiles per head whose maxima the cut search holds in registers (per
// lane 32; beyond that it reads the staged copy on every step), and the low
// key bits the register search leaves zero (its cut is then at most 2^-11
// relative below the exact K-th tile maximum: a few more candidates, the
// same selection).
constexpr int kSelRegs = 32;
constexpr int kCutLowBits = 12;

// Sum of v over the wave, in every lane (DPP row rotations and lane-half
// swaps, no LDS).
__device__ inline int wave_sum_i32(int v) {
    v += (int)row_ror<1>((uint32_t)v);
    v += (int)row_ror<2>((uint32_t)v);
    v += (int)row_ror<4>((uint32_t)v);
    v += (int)row_ror<8>((uint32_t)v);
    LanePair p = swap16((uint32_t)v);
    v = (int)p.a + (int)p.b;
    p = swap32((uint32_t)v);
    return (int)p.a + (int)p.b;
}

// Largest uint32 over the wave, in every lane (DPP row rotations and
// lane-half swaps, no LDS).
__device__ inline uint32_t wave_max_u32(uint32_t v) {
    v = max(v, row_ror<1>(v));
    v = max(v, row_ror<2>(v));
    v = max(v, row_ror<4>(v));
    v = max(v, row_ror<8>(v));
    LanePair p = swap16(v);
    v = max(p.a, p.b);
    p = swap32(v);
    return max(p.a, p.b);
}

// fp32 -> uint32 with the same order (no NaN among scores) and back.
__device__ inline uint32_t fkey(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ inline float unfkey(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k); }

// The score MFMA's B operand of the wave's head quad: head j = lane % 4 of
// the quad, dims 4s..4s+3 (heads past the group read the group's first
// head, as the attention kernel does; their scores are never kept).
template <int D>
__device__ inline void load_qv(const SelectArgs& a, int64_t o0, int quad, int lane, fkv_h4 (&qv)[D / 4]) {
    const int j = lane & 3;
    const uint16_t* qrow = a.q + (4 * quad + j < a.G ? o0 + j : o0 - 4 * quad) * D;
#pragma unroll
    for (int s = 0; s < D / 4; s++) {
        uint2 w;
        __builtin_memcpy(&w, qrow + 4 * s, 8);
        qv[s] = __builtin_bit_cast(fkv_h4, w);
    }
}

// The far tiles' 64 scores for the wave's head quad as the attention
// kernel computes them: lane = token 4 blk + e of the tile, e = 0..3, head
// lane % 4 (the same E4M3 operands, fp16 query and MFMA chain in the same
// order: the same fp32 bits).  N tiles, all loads issued before any MFMA.
template <int D, int N>
__device__ inline void rescore_tiles(const SelectArgs& a, int64_t bkv, const int (&tile)[N],
                                     const fkv_h4 (&qv)[D / 4], float far_scale, int lane, float (&sv)[N][4]) {
    uint4 kc[N][D / 16];
#pragma unroll
    for (int n = 0; n < N; n++) {
        const uint8_t* rec = a.blob + a.L.far + far_rec_index(a.L, bkv, tile[n]) * (int64_t)a.L.far_rec;
#pragma unroll
        for (int c = 0; c < D / 16; c++) kc[n][c] = *(const uint4*)(rec + c * 1024 + lane * 16);
    }
    // one round trip for the batch: every load is issued before the first
    // use (the compiler would otherwise hoist the first conversions and
    // MFMAs between the loads and wait for the first ones early); nothing
    // is scheduled across the barrier
    __builtin_amdgcn_sched_barrier(0);
    fkv_f4 acc[N];
#pragma unroll
    for (int n = 0; n < N; n++) acc[n] = fkv_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 4; s++)
#pragma unroll
        for (int n = 0; n < N; n++) acc[n] = mfma4_local(e4m3x4(word_of(kc[n][s >> 2], s & 3)), qv[s], acc[n]);
#pragma unroll
    for (int n = 0; n < N; n++)
#pragma unroll
        for (int e = 0; e < 4; e++) sv[n][e] = acc[n][e] * far_scale;
}

// (s, t) ahead of (s2, t2): higher score, or equal and the smaller token.
__device__ inline bool ahead_of(float s, int t, float s2, int t2) { return s > s2 || (s == s2 && t < t2); }

// Insert (s, t) into a list held in lanes 0..K-1 (n entries, in order);
// the whole wave calls it with the same (s, t).
__device__ inline void list_insert(float& ls, int& li, int& n, int K, float s, int t, int lane) {
    const bool ahead = lane < n && ahead_of(ls, li, s, t);
    const int pos = __builtin_popcountll(__builtin_amdgcn_ballot_w64(ahead));
    if (pos >= K) return;
    const float ps = __shfl_up(ls, 1);
    const int pi = __shfl_up(li, 1);
    if (lane > pos) {
        ls = ps;
        li = pi;
    } else if (lane == pos) {
        ls = s;
        li = t;
    }
    n = n < K ? n + 1 : K;
}

// One (score, token) per lane sorted across the wave, best first (bitonic
// network on lane swaps; equal pairs are the padding (-inf, INT_MAX)).
__device__ inline void wave_sort(float& s, int& t, int lane) {
#pragma unroll
    for (int k = 2; k <= kWave; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const float ps = __shfl_xor(s, j);
            const int pt = __shfl_xor(t, j);
            const bool pb = ahead_of(ps, pt, s, t);
            const bool lower = (lane & j) == 0, want = (lane & k) == 0;
            if (lower == want ? pb : ahead_of(s, t, ps, pt)) {
                s = ps;
                t = pt;
            }
        }
}

// The cut of one head from its NSL x 64 tile maxima (tm, ntf of them; the
// wave of the head): the largest key x with its low kCutLowBits bits zero
// that at least K maxima above th reach (at most the K-th largest), or
// -inf when at most K maxima clear th.  The maxima are held as keys in
// registers (0 for those at or below th, or past the far tier: below every
// trial) and copied to the LDS row `lds` (NSL x 64 entries, -inf past the
// far tier) for the rescoring.  raw: the lane's maxima r * 64 + lane, loaded
// at the kernel's entry by buffer loads bounded by the far tier (past it
// they read 0 without touching memory), so none sits behind a branch and
// all are in flight at once (guarded loads had been compiled as one
// branch, load and wait each, a round trip per 64 tiles).
// A count is one compare and add per register and one wave sum on DPP
// (per-register ballots, each a vector-to-scalar round trip through VCC,
// were twice as slow per step).
template <int NSL>
__device__ inline float cut_search(const uint32_t (&raw)[kSelRegs], int ntf, float th, int K, int lane, float* lds) {
    uint32_t kv[NSL];
#pragma unroll
    for (int r = 0; r < NSL; r++) {
        const int t = r * kWave + lane;
        const float v = t < ntf ? __uint_as_float(raw[r]) : -INFINITY;
        lds[t] = v;
        kv[r] = v > th ? fkey(v) : 0u;
    }
    auto count_at_least = [&](uint32_t trial) {
        int c = 0;
#pragma unroll
        for (int r = 0; r < NSL; r++) c += kv[r] >= trial ? 1 : 0;
        return __builtin_amdgcn_readfirstlane(wave_sum_i32(c));
    };
    if (count_at_least(1u) <= K) return -INFINITY;
    // every key above th lies in [fkey(th) + 1, the largest key]: the bits
    // above the highest one where the two bounds differ are the cut's too
    // (a trial with such a bit set counts every key or none), so the
    // search starts below them
    uint32_t kmax = 0;
#pragma unroll
    for (int r = 0; r < NSL; r++) kmax = kv[r] > kmax ? kv[r] : kmax;
    kmax = __builtin_amdgcn_readfirstlane(wave_max_u32(kmax));
    const uint32_t diff = (fkey(th) + 1u) ^ kmax;
    const int top = diff ? 31 - __builtin_clz(diff) : -1;  // the highest differing bit
    uint32_t x = top < 0 ? kmax : top >= 31 ? 0u : kmax & ~((2u << top) - 1u);
    x &= ~((1u << kCutLowBits) - 1u);
    for (int bit = top < 31 ? top : 31; bit >= kCutLowBits; bit--) {
        const uint32_t trial = x | (1u << bit);
        if (count_at_least(trial) >= K) x = trial;
    }
    return unfkey(x);  // x >= the key of -FLT_MAX: a finite cut
}

// Top-K spike selection, part 2, for head `wave` of a quad, run by the
// last workgroup of the quad to finish part 1 (spike_candidates_kernel):
// keeps the best K of the head's candidates in lanes 0..K-1 (the first 64
// sorted across the wave, the rest inserted), writes the outputs and
// re-arms the head's candidate count.  The candidates of the other
// workgroups are read with sc1 loads (coherent across XCDs), the count
// with an agent-scope atomic load.  A buffer (64 K pairs) overflows only
// when more than K tiles reach the cut: ties at the K-th largest maximum,
// or, after the register cut search, maxima less than 2^-11 relative below
// it; that head then re-scans its tiles itself.  Output: flags = the spike
// count (at most K), tokens[0..count) the list; entry 0 is the attention
// kernel's first-index argmax when nothing spikes (the reference's single
// token), the rest -1.
template <int D>
__device__ inline void select_head(const SelectArgs& a, int quad, int kvh, int b, int wave, int lane, float cut) {
    const int j = lane & 3, blk = lane >> 2;
    if (4 * quad + wave >= a.G) return;
    const int64_t bkv = (int64_t)b * a.L.Hkv + kvh;
    const int64_t o0 = (int64_t)b * a.Hq + (int64_t)kvh * a.G + 4 * quad, oj = o0 + wave;
    const int K = a.K;
    float ls = -INFINITY;
    int li = INT_MAX, n = 0;
    if (a.flags_in[oj] != 0) {
        // the first 64 pairs are loaded together with the count (one round
        // trip); loads past the head's buffer read 0
        const __amdgpu_buffer_rsrc_t rs_s =
            __builtin_amdgcn_make_buffer_rsrc((void*)(a.cand_s + oj * a.cap), (short)0, a.cap * 4, 0x00020000);
        const __amdgpu_buffer_rsrc_t rs_t =
            __builtin_amdgcn_make_buffer_rsrc((void*)(a.cand_t + oj * a.cap), (short)0, a.cap * 4, 0x00020000);
        const uint32_t rs0 = __builtin_amdgcn_raw_buffer_load_b32(rs_s, lane * 4, 0, kCpolSc1);
        const uint32_t rt0 = __builtin_amdgcn_raw_buffer_load_b32(rs_t, lane * 4, 0, kCpolSc1);
        const int nb = __builtin_amdgcn_readfirstlane(
            __hip_atomic_load(a.cand_n + oj, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (nb <= kWave) {
            // each pair's place in the list = the pairs ahead of it (distinct
            // tokens: a strict order); a forward permute puts rank p in lane
            // p (lanes past nb keep their own place)
            const float s = lane < nb ? __uint_as_float(rs0) : -INFINITY;
            const int t = lane < nb ? (int)rt0 : INT_MAX;
            int r = 0;
            for (int src = 0; src < nb; src++) {
                const float ss = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), src));
                const int ts = __builtin_amdgcn_readlane(t, src);
                r += ahead_of(ss, ts, s, t) ? 1 : 0;
            }
            if (lane >= nb) r = lane;
            ls = __int_as_float(__builtin_amdgcn_ds_permute(r * 4, __float_as_int(s)));
            li = __builtin_amdgcn_ds_permute(r * 4, t);
            n = nb < K ? nb : K;
        } else if (nb <= a.cap) {
            for (int c0 = 0; c0 < nb; c0 += kWave) {
                const int i = c0 + lane;
                const uint32_t rsv = c0 == 0 ? rs0 : __builtin_amdgcn_raw_buffer_load_b32(rs_s, i * 4, 0, kCpolSc1);
                const uint32_t rtv = c0 == 0 ? rt0 : __builtin_amdgcn_raw_buffer_load_b32(rs_t, i * 4, 0, kCpolSc1);
                float s = i < nb ? __uint_as_float(rsv) : -INFINITY;
                int t = i < nb ? (int)rtv : INT_MAX;
                if (c0 == 0) {  // the first 64: one sort, the best K become the list
                    wave_sort(s, t, lane);
                    ls = s;
                    li = t;
                    n = K;
                    continue;
                }
                const float ks = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ls), K - 1));
                const int kt = __builtin_amdgcn_readlane(li, K - 1);
                uint64_t m = __builtin_amdgcn_ballot_w64(i < nb && (n < K || ahead_of(s, t, ks, kt)));
                while (m) {
                    const int src = (int)__builtin_ctzll(m);
                    m &= m - 1;
                    list_insert(ls, li, n, K, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), src)),
                                __builtin_amdgcn_readlane(t, src), lane);
                }
            }
        } else {
            // more than K tiles reached the cut: this head re-scans its tiles
            fkv_h4 qv[D / 4];
            load_qv<D>(a, o0, quad, lane, qv);
            const float far_scale = a.inv_sqrt_d * (a.kscale ? a.kscale[bkv] : 1.0f);
            const float thj = a.thr[oj], ctj = cut;
            const float* tm = a.tmax + oj * a.ntf;
            for (int c0 = 0; c0 < a.ntf; c0 += kWave) {
                const int tl = c0 + lane;
                const bool cand = tl < a.ntf && tm[tl] > thj && tm[tl] >= ctj;
                uint64_t mask = __builtin_amdgcn_ballot_w64(cand);
                while (mask) {
                    const int tile[1] = {c0 + (int)__builtin_ctzll(mask)};
                    mask &= mask - 1;
                    float sv[1][4];
                    rescore_tiles<D, 1>(a, bkv, tile, qv, far_scale, lane, sv);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int t0 = tile[0] * kTile + e;
                        uint64_t m = __builtin_amdgcn_ballot_w64(j == wave && t0 + 4 * blk < a.L.F &&
                                                                  sv[0][e] > thj && sv[0][e] >= ctj);
                        while (m) {
                            const int src = (int)__builtin_ctzll(m);
                            m &= m - 1;
                            list_insert(ls, li, n, K,
                                        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv[0][e]), src)),
                                        t0 + 4 * (src >> 2), lane);
                        }
                    }
                }
            }
        }
    }
    if (lane < K) {
        int t = lane < n ? li : -1;
        if (lane == 0 && n == 0) t = a.tokens_in[oj];
        a.tokens[oj * K + lane] = t;
    }
    if (lane == 0) {
        a.flags[oj] = n;
        __hip_atomic_store(a.cand_n + oj, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // re-armed for the next call
    }
}

// Top-K spike selection, part 1: kSelParts workgroups per (batch, KV head,
// head quad).  A far token spikes when its score exceeds its head's
// threshold min_near + margin (the attention kernel's flag rule); each head
// reports its best K spiking tokens, score descending, ties to the smaller
// index.  The K best tokens lie in the K far tiles of highest maximum
// (among the tiles whose maximum clears the threshold): a tile holding one
// of them has a maximum at least that token's score, and at most K - 1
// tokens -- so at most K - 1 tiles -- score higher.  So, from the tile
// maxima the attention kernel stored:
//  A. wave j finds head j's cut, the K-th largest tile maximum above the
//     threshold (a bitwise binary search on order-preserving keys), or -inf
//     when at most K tiles clear the threshold (every workgroup of the
//     quad computes the same cuts);
//  B. the quad's kSelParts x 4 waves share out the tiles whose maximum
//     clears some head's threshold and cut by their rank in tile order
//     (each 64-tile chunk's candidate mask computed once per workgroup,
//     in LDS; wave gw takes ranks gw, gw + kSelParts * 4, ...), rescore
//     them four at a time (rescore_tiles: the attention kernel's bits) and
//     append every token
//     above its head's threshold and at or above its cut to the head's
//     candidate buffer in memory -- at least K tokens when the cut is set
//     (each of the K tiles contributes its maximum), all of them
//     otherwise, at most 64 per tile at or above the cut;
//  C. the last workgroup of the quad to finish B (an arrival count per
//     quad, re-armed by that workgroup) runs part 2, select_head, for the
//     quad's heads.  Candidate pairs are written with sc1 stores (coherent
//     across XCDs) and a workgroup's arrival is counted once its stores are
//     complete.  A quad where nothing spikes skips B and C: its first
//     workgroup writes the outputs.
template <int D>
__global__ __launch_bounds__(64 * kSelWaves) void spike_candidates_kernel(SelectArgs a) {
    constexpr int NS = D / 4, NR = 4;  // tiles rescored together
    __shared__ float thr_s[4], cut_s[4];
    __shared__ int fl_s[4], last_s;
    __shared__ uint64_t cmask_s[kSelStage / kWave];  // candidate tiles per 64-tile chunk (staged tiers)
    __shared__ float tm_s[4][kSelStage];
    const int quad = blockIdx.x / kSelParts, part = blockIdx.x % kSelParts, kvh = blockIdx.y, b = blockIdx.z;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave), lane = threadIdx.x % kWave;
    const int j = lane & 3, blk = lane >> 2;
    const int64_t bkv = (int64_t)b * a.L.Hkv + kvh;
    const int64_t o0 = (int64_t)b * a.Hq + (int64_t)kvh * a.G + 4 * quad;  // head 0 of the quad
    const int K = a.K, ntf = a.ntf;
    const bool staged = ntf <= kSelStage;
    FKV_SEL_STAMP(threadIdx.x == 0, 0);
    // the rescoring's query operands and (tiers of at most kSelRegs x 64
    // tiles) the cut search's tile maxima, head `wave`'s, in flight with the
    // thresholds' and flags' loads
    fkv_h4 qv[NS];
    load_qv<D>(a, o0, quad, lane, qv);
    const bool regs = ntf <= kWave * kSelRegs;
    uint32_t tmr[kSelRegs];
    {
        const bool own = regs && 4 * quad + wave < a.G;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.tmax + (o0 + wave) * ntf), (short)0, own ? ntf * 4 : 0, 0x00020000);
#pragma unroll
        for (int r = 0; r < kSelRegs; r++) tmr[r] = __builtin_amdgcn_raw_buffer_load_b32(rs, (r * kWave + lane) * 4, 0, 0);
    }
    if (threadIdx.x < 4) {
        const int jj = threadIdx.x;
        const bool live = 4 * quad + jj < a.G;
        thr_s[jj] = live ? a.thr[o0 + jj] : INFINITY;
        fl_s[jj] = live && a.flags_in[o0 + jj] != 0;
        cut_s[jj] = INFINITY;
    }
    __syncthreads();
    if (!(fl_s[0] | fl_s[1] | fl_s[2] | fl_s[3])) {  // nothing spikes: the outputs only
        if (part == 0) select_head<D>(a, quad, kvh, b, wave, lane, INFINITY);
        return;
    }
    // the register path: each flagged head's wave writes the LDS copy of its
    // maxima that the rescoring reads in the cut search below
    // the tile maxima of the quad's heads that exist (4 quad + jj < G) as one
    // bounded buffer: loads past them read 0 without touching memory, so
    // none needs a branch (a guarded load compiles to a branch, the load and
    // a wait of its own)
    const int live = min(4, a.G - 4 * quad);
    const __amdgpu_buffer_rsrc_t qrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.tmax + o0 * ntf), (short)0, live * ntf * 4, 0x00020000);
    // otherwise the tile maxima of the quad's flagged heads -> LDS, eight loads in flight per thread
    if (staged && !regs) {
        constexpr int U = 8;
        for (int i0 = threadIdx.x; i0 < 4 * ntf; i0 += U * (int)blockDim.x) {
            uint32_t raw[U];
#pragma unroll
            for (int u = 0; u < U; u++)
                raw[u] = __builtin_amdgcn_raw_buffer_load_b32(qrs, (i0 + u * (int)blockDim.x) * 4, 0, 0);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = i0 + u * (int)blockDim.x, jj = i / ntf;
                if (i < 4 * ntf) tm_s[jj][i % ntf] = fl_s[jj] ? __uint_as_float(raw[u]) : -INFINITY;
            }
        }
    }
    __syncthreads();
    FKV_SEL_STAMP(threadIdx.x == 0, 1);
    auto tmv = [&](int jj, int t) -> float { return staged ? tm_s[jj][t] : a.tmax[(o0 + jj) * ntf + t]; };
    // ---- A: head `wave`'s cut ----
    if (wave < 4 && fl_s[wave]) {
        const float th = thr_s[wave];
        float cut = -INFINITY;
        if (regs) {
            if (ntf <= 8 * kWave) cut = cut_search<8>(tmr, ntf, th, K, lane, tm_s[wave]);
            else if (ntf <= 16 * kWave) cut = cut_search<16>(tmr, ntf, th, K, lane, tm_s[wave]);
            else cut = cut_search<kSelRegs>(tmr, ntf, th, K, lane, tm_s[wave]);
        } else {
            int above = 0;
            for (int t = lane; t < ntf; t += kWave) above += tmv(wave, t) > th;
            for (int o = 32; o >= 1; o >>= 1) above += __shfl_xor(above, o);
            if (above > K) {
                uint32_t x = 0;
                for (int bit = 31; bit >= 0; bit--) {
                    const uint32_t trial = x | (1u << bit);
                    int c = 0;
                    for (int t = lane; t < ntf; t += kWave) {
                        const float v = tmv(wave, t);
                        c += v > th && fkey(v) >= trial;
                    }
                    for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o);
                    if (c >= K) x = trial;
                }
                cut = unfkey(x);
            }
        }
        if (lane == 0) cut_s[wave] = cut;
    }
    __syncthreads();
    FKV_SEL_STAMP(threadIdx.x == 0, 2);
    float th[4], ct[4];
    int fl[4];
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        th[jj] = thr_s[jj];
        ct[jj] = cut_s[jj];
        fl[jj] = fl_s[jj];
    }
    const float far_scale = a.inv_sqrt_d * (a.kscale ? a.kscale[bkv] : 1.0f);
    FKV_SEL_STAMP(lane == 0, 7 + wave);
    // the quad's candidate pairs (heads that exist) as bounded buffers
    const __amdgpu_buffer_rsrc_t cs_rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.cand_s + o0 * a.cap), (short)0, live * a.cap * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t ct_rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.cand_t + o0 * a.cap), (short)0, live * a.cap * 4, 0x00020000);
    // ---- B: this wave's candidate tiles (every kSelParts * kSelWaves-th), NR at a time ----
    const int gw = part * kSelWaves + wave, nw = kSelParts * kSelWaves;
    int np = 0;  // tiles pending
    int nfl = 0;        // batches flushed (the phase stamps time the first)
    (void)nfl;
    int pend[NR];
#pragma unroll
    for (int n = 0; n < NR; n++) pend[n] = -1;
    auto flush = [&](int count) __attribute__((always_inline)) {
        int tl[NR];
#pragma unroll
        for (int n = 0; n < NR; n++) tl[n] = n < count ? pend[n] : pend[0];
        float sv[NR][4];
        FKV_SEL_STAMP(lane == 0 && nfl == 0, 16 + wave);
        rescore_tiles<D, NR>(a, bkv, tl, qv, far_scale, lane, sv);
        FKV_SEL_STAMP(lane == 0 && nfl == 0, 20 + wave);
        // the lane's candidates of the batch
        uint32_t pm = 0;
#pragma unroll
        for (int n = 0; n < NR; n++) {
            if (n >= count) break;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = tl[n] * kTile + 4 * blk + e;
                if (fl[j] && t < a.L.F && sv[n][e] > th[j] && sv[n][e] >= ct[j]) pm |= 1u << (4 * n + e);
            }
        }
        // one atomic per head and batch: a lane's slots follow those of the
        // lanes of its head (lane % 4 == j) below it; its offset and the
        // head's total come from bit-sliced ballots of the counts (0..16)
        const int cnt = __builtin_popcount(pm);
        const uint64_t head_lanes = 0x1111111111111111ull << j;
        const uint64_t below = lane ? ~0ull >> (64 - lane) : 0ull;
        int pre = 0, tot = 0;
#pragma unroll
        for (int b = 0; b < 5; b++) {
            const uint64_t m = __builtin_amdgcn_ballot_w64((cnt >> b) & 1) & head_lanes;
            pre += __builtin_popcountll(m & below) << b;
            tot += __builtin_popcountll(m) << b;
        }
        int base = 0;
        if (lane < 4 && tot > 0) base = atomicAdd(a.cand_n + o0 + lane, tot);  // lane j < 4: head j
        const int b0 = __builtin_amdgcn_readlane(base, 0), b1 = __builtin_amdgcn_readlane(base, 1);
        const int b2 = __builtin_amdgcn_readlane(base, 2), b3 = __builtin_amdgcn_readlane(base, 3);
        FKV_SEL_STAMP(lane == 0 && nfl == 0, 24 + wave);
        nfl++;
        if (pm == 0) return;
        int slot = (j == 0 ? b0 : j == 1 ? b1 : j == 2 ? b2 : b3) + pre;
#pragma unroll
        for (int n = 0; n < NR; n++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                if ((pm >> (4 * n + e)) & 1u) {
                    if (slot < a.cap) {
                        const int off = (j * a.cap + slot) * 4;
                        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sv[n][e]), cs_rs, off, 0, kCpolSc1);
                        __builtin_amdgcn_raw_buffer_store_b32((uint32_t)(tl[n] * kTile + 4 * blk + e), ct_rs, off, 0,
                                                              kCpolSc1);
                    }
                    slot++;
                }
    };
    // queue one of this wave's tiles; a full batch is rescored at once
    auto take = [&](int tile) __attribute__((always_inline)) {
#pragma unroll
        for (int n = 0; n < NR; n++)
            if (n == np) pend[n] = tile;
        if (++np == NR) {
            flush(NR);
            np = 0;
        }
    };
    if (staged) {
        // B1: each 64-tile chunk's candidate tiles as a mask, the chunks
        // shared among the workgroup's waves (at most 64 chunks)
        const int nch = (ntf + kWave - 1) / kWave;
        for (int c = wave; c < nch; c += kSelWaves) {
            const int tl = c * kWave + lane;
            float v[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) v[jj] = tm_s[jj][tl < ntf ? tl : 0];
            bool cand = false;
            if (tl < ntf) {
#pragma unroll
                for (int jj = 0; jj < 4; jj++) cand |= fl[jj] && v[jj] > th[jj] && v[jj] >= ct[jj];
            }
            const uint64_t m = __builtin_amdgcn_ballot_w64(cand);
            if (lane == 0) cmask_s[c] = m;
        }
        __syncthreads();
        // B2: lane c holds chunk c's mask and the candidates of the chunks
        // before it (a bit-sliced prefix count: one ballot per count bit);
        // candidate rho (in tile order) is the nth set bit of its chunk's
        // mask, found by the lane whose bit it is
        const uint64_t mc = lane < nch ? cmask_s[lane] : 0ull;
        const int cnt = (int)__builtin_popcountll(mc);
        int excl = 0;
#pragma unroll
        for (int bb = 0; bb < 7; bb++) {
            const uint64_t bm = __builtin_amdgcn_ballot_w64((cnt >> bb) & 1);
            excl += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0u))
                    << bb;
        }
        const int total = __builtin_amdgcn_readlane(excl + cnt, kWave - 1);
        for (int rho = gw; rho < total; rho += nw) {
            const int c = (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(excl + cnt > rho));
            const int nth = rho - __builtin_amdgcn_readlane(excl, c);
            const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)mc, c);
            const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(mc >> 32), c);
            const uint64_t m = ((uint64_t)hi << 32) | lo;
            const bool hit = ((m >> lane) & 1ull) &&
                             (int)__builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0u)) == nth;
            take(c * kWave + (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(hit)));
        }
    } else {
        // far tiers past the LDS stage: one chunk at a time, the maxima read
        // from memory; the wave takes the candidates whose rank (in tile
        // order) is gw mod nw
        int r = 0;  // candidates seen (the same in every wave of the quad)
        for (int c0 = 0; c0 < ntf; c0 += kWave) {
            const int tl = c0 + lane;
            float v[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const uint32_t raw = __builtin_amdgcn_raw_buffer_load_b32(qrs, (jj * ntf + tl) * 4, 0, 0);
                v[jj] = fl[jj] && tl < ntf ? __uint_as_float(raw) : -INFINITY;
            }
            bool cand = false;
            if (tl < ntf) {
#pragma unroll
                for (int jj = 0; jj < 4; jj++) cand |= fl[jj] && v[jj] > th[jj] && v[jj] >= ct[jj];
            }
            const uint64_t mask = __builtin_amdgcn_ballot_w64(cand);
            const int rank = r + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
            uint64_t mine = __builtin_amdgcn_ballot_w64(cand && rank % nw == gw);
            r += (int)__builtin_popcountll(mask);
            while (mine) {
                const int bit = (int)__builtin_ctzll(mine);
                mine &= mine - 1;
                take(c0 + bit);
            }
        }
    }
    FKV_SEL_STAMP(lane == 0, 11 + wave);
    if (np > 0) flush(np);
    FKV_SEL_STAMP(lane == 0, 3 + wave);
    // ---- C: the quad's last workgroup selects ----
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this workgroup's pairs are stored
    __syncthreads();
    const int64_t qrow = bkv * (int64_t)(gridDim.x / kSelParts) + quad;
    if (threadIdx.x == 0)
        last_s = __hip_atomic_fetch_add(a.arrive + qrow, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 kSelParts - 1;
    __syncthreads();
    if (!last_s) return;
    select_head<D>(a, quad, kvh, b, wave, lane, cut_s[wave]);
    if (threadIdx.x == 0) __hip_atomic_store(a.arrive + qrow, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    FKV_SEL_STAMP(lane == 0, 15);
}

// ---------------------------------------------------------------------------
// Promotion, GPU side (csrc/promotion_pipeline.cpp:192-241): exact fp16 rows
// into near-tier headroom slots, then the near_valid bump
// ---------------------------------------------------------------------------

// One workgroup per promoted row: record i = (head, slot) = hs[2i], hs[2i+1];
// rows_k / rows_v hold [n][nb][D] fp16 for batches 0..nb-1 (the same slot in
// every batch: near_valid is shared across the batch; batches without an
// archive row keep their slot as it is, as the reference's batch-0-only
// copy does).  Records outside the blob are skipped.
__global__ void promote_rows_kernel(const int32_t* __restrict__ hs, const uint16_t* __restrict__ rows_k,
                                    const uint16_t* __restrict__ rows_v, int n, int nb, BlobLayout L,
                                    uint8_t* __restrict__ blob) {
    const int i = blockIdx.x;
    if (i >= n) return;
    const int h = hs[2 * i], slot = hs[2 * i + 1];
    if (h < 0 || h >= L.Hkv || slot < 0 || slot >= L.Na) return;
    uint16_t* nk = (uint16_t*)(blob + L.near_k);
    uint16_t* nv = (uint16_t*)(blob + L.near_v);
    for (int e = threadIdx.x; e < nb * L.D; e += blockDim.x) {
        const int b = e / L.D, d = e % L.D;
        const int64_t base = ((int64_t)b * L.Hkv + h) * L.Na_pad * L.D;
        const int64_t src = ((int64_t)i * nb + b) * L.D + d;
        nk[base + near_k_index(slot, d, L.D)] = rows_k[src];
        nv[base + near_v_index(slot, d, L.D)] = rows_v[src];
    }
}

// After the rows (stream order): near_valid[h] = max(near_valid[h], slot + 1)
// for every record, as device-scope atomics.
__global__ void bump_near_valid_kernel(const int32_t* __restrict__ hs, int n, BlobLayout L, uint8_t* blob) {
    unsigned* valid = (unsigned*)(blob + L.near_valid);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int h = hs[2 * i], slot = hs[2 * i + 1];
        if (h < 0 || h >= L.Hkv || slot < 0 || slot >= L.Na) continue;
        atomicMax(valid + h, (unsigned)(slot + 1));
    }
}

// Near tier of the blob back to row-major (B, Hkv, Na, D) fp16.
__global__ void export_near_kernel(BlobLayout L, const uint8_t* __restrict__ blob, uint16_t* __restrict__ ok,
                                   uint16_t* __restrict__ ov) {
    const int64_t n = (int64_t)L.B * L.Hkv * L.Na * L.D;
    const uint16_t* nk = (const uint16_t*)(blob + L.near_k);
    const uint16_t* nv = (const uint16_t*)(blob + L.near_v);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int d = (int)(i % L.D);
        const int t = (int)((i / L.D) % L.Na);
        const int64_t bkv = i / ((int64_t)L.D * L.Na);
        const int64_t base = bkv * L.Na_pad * L.D;
        if (ok) ok[i] = nk[base + near_k_index(t, d, L.D)];
        if (ov) ov[i] = nv[base + near_v_index(t, d, L.D)];
    }
}

__global__ void zero_ints_kernel(int* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

}  // namespace fkv

// ---------------------------------------------------------------------------
// Host side: handle + launch
// ---------------------------------------------------------------------------

namespace fkv {

// TurboQuant attention kernels (fmt 1), instantiated in this translation
// unit (default instruction scheduling); the fp8 and group-32 ones come
// from attn_kernel_one_quad / attn_kernel_quads.
template <int D>
static AttnKernel pick_attn_turbo(int nq) {
    switch (nq) {
        case 1: return attn_kernel<D, 1, 1>;
        case 2: return attn_kernel<D, 2, 1>;
        case 3: return attn_kernel<D, 3, 1>;
        default: return attn_kernel<D, 4, 1>;
    }
}

int grid_for(int64_t n, int block) {
    int64_t g = cdiv(n, block);
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (int)g;
}

static int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// Workgroups per (b, kv_head, head group): enough to fill 256 CUs, at least
// two tiles per wave.
static int plan_splits(const BlobLayout& L, int rows, int n_dec, int target, int waves = kWavesPerGroup) {
    const int tiles = (int)(cdiv(L.Na, kTile) + cdiv(L.F, kTile) + cdiv(n_dec, kTile));
    int s = (int)cdiv(target, rows > 0 ? rows : 1);
    const int cap = tiles / (2 * waves);
    if (s > cap) s = cap;
    if (s > kMaxSplits) s = kMaxSplits;
    return s < 1 ? 1 : s;
}

static size_t partial_floats(int rows, int splits, int ng_max, int D) {
    return (size_t)rows * splits * ng_max * (kHdr + D);
}

// Query heads per workgroup row: the whole GQA group (up to kHeads), so
// every compressed byte crosses HBM once -- unless that leaves most CUs idle
// (few batch x KV-head rows, short context): then rows of 4 heads, more
// workgroups re-reading the same small KV from L2.
LaunchPlan plan_launch(const BlobLayout& L, int Hq, int n_decode, int target_wgs) {
    const int G = Hq / L.Hkv;
    int hpg = kHeads;
    const int rows16 = L.B * L.Hkv * (int)cdiv(G, kHeads);
    if (G > 4 && rows16 * plan_splits(L, rows16, n_decode, target_wgs) < kSmallGrid) hpg = 4;
    LaunchPlan p;
    p.hpg = hpg;
    p.head_groups = (int)cdiv(G, hpg);
    p.ng_max = G < hpg ? G : hpg;
    p.rows = L.B * L.Hkv * p.head_groups;
    p.waves = attn_waves(L.D, (int)cdiv(p.ng_max, 4), L.fmt);
    p.splits = plan_splits(L, p.rows, n_decode, target_wgs, p.waves);
    // rows of 2..4 splits keep one record per wave (their merge reads at most
    // 16 records, 32 for 8-wave TurboQuant rows: within kMaxSplits); rows of
    // more splits merge their waves in LDS first (C4's 8 splits: 32 wave
    // records merged 0.4 us slower than 8 merged records)
    p.wave_recs = p.splits > 1 && p.splits <= 4 ? p.waves : 1;
    p.ws_floats = p.splits > 1 ? partial_floats(p.rows, p.splits * p.wave_recs, p.ng_max, L.D) : 0;
    return p;
}

// Both row widths at the largest record count per row (64: kMaxSplits
// merged records, or 16 splits of 4 wave records): covers plan_launch for
// every decode length and target.
size_t workspace_floats(const BlobLayout& L, int Hq) {
    const int G = Hq / L.Hkv;
    size_t best = 0;
    for (int hpg : {4, kHeads}) {
        const size_t f = partial_floats(L.B * L.Hkv * (int)cdiv(G, hpg), kMaxSplits, G < hpg ? G : hpg, L.D);
        best = f > best ? f : best;
    }
    return best;
}

int workspace_rows(const BlobLayout& L, int Hq) { return L.B * L.Hkv * (int)cdiv(Hq / L.Hkv, 4); }

}  // namespace fkv

using fkv::check_hip;
using fkv::set_error;

namespace fkv {

// ---------------------------------------------------------------------------
// The workgroup -> XCD dispatch rule, checked once per device: a probe
// dispatch records the XCD (HW_REG_XCC_ID) of each of its workgroups; the
// rule holds when, with the XCDs numbered x0 .. x0 + X - 1, workgroup i ran
// on x0 + (c + i) mod X for one offset c.  X then enables the XCD-local
// split merge; otherwise the merge goes through memory.  The probe writes
// a file-scope device array (no allocation).
// ---------------------------------------------------------------------------

constexpr int kXcdProbeWGs = 4096;
constexpr int kXcdDevices = 64;
static __device__ uint32_t xcd_probe_out[kXcdProbeWGs];

__global__ void xcd_probe_kernel(uint32_t* out) {
    const uint32_t x = xcc_id();
    if (threadIdx.x == 0) out[blockIdx.x] = x;
}

namespace {
std::mutex g_xcd_mu;
struct XcdRule {
    bool done = false;
    int mod = 0;
};
XcdRule g_xcd[kXcdDevices];
}  // namespace

int xcd_rule(int dev, hipStream_t st, int* mod) {
    if (dev < 0 || dev >= kXcdDevices) return set_error("xcd_rule: device index out of range");
    std::lock_guard<std::mutex> lock(g_xcd_mu);
    XcdRule& r = g_xcd[dev];
    if (!r.done) {
        void* out = nullptr;
        if (int rc = check_hip(hipGetSymbolAddress(&out, HIP_SYMBOL(xcd_probe_out)), "hipGetSymbolAddress(xcd_probe_out)"))
            return rc;
        if (!out) return set_error("xcd_rule: hipGetSymbolAddress returned NULL");
        hipLaunchKernelGGL(xcd_probe_kernel, dim3(kXcdProbeWGs), dim3(kWave), 0, st, (uint32_t*)out);
        std::vector<uint32_t> x(kXcdProbeWGs);
        int rc = check_hip(hipGetLastError(), "xcd_probe_kernel launch");
        if (!rc) rc = check_hip(hipMemcpyAsync(x.data(), out, kXcdProbeWGs * sizeof(uint32_t), hipMemcpyDeviceToHost, st),
                                "hipMemcpyAsync(xcd probe)");
        if (!rc) rc = check_hip(hipStreamSynchronize(st), "hipStreamSynchronize");
        if (rc) return rc;
        int32_t X = 0, c = 0;
        (void)fkv_xcd_rule_fit(x.data(), kXcdProbeWGs, &X, &c);
        r.mod = X;
        r.done = true;
    }
    *mod = r.mod;
    return FKV_OK;
}

int attn_begin(fkv_attn_impl* h, int B, int Hkv, int D, int Na, int F, int fmt, const void* near_k,
               const void* near_v, int near_dtype, const int32_t* near_valid, float margin, hipStream_t st) {
    h->L = make_layout(B, Hkv, D, Na, F, fmt);
    h->margin = margin;
    // tuning knobs are read once here, never on the call path
    h->target_wgs = env_int("FKV_TARGET_WGS", 256);
    if (h->target_wgs < 1) h->target_wgs = 1;
    h->fused_merge = env_int("FKV_FUSED_MERGE", 1) != 0;
    int rc = check_hip(hipGetDevice(&h->device), "hipGetDevice");
    if (!rc) rc = check_hip(hipMalloc(&h->blob, h->L.total), "hipMalloc(blob)");
    if (!rc) rc = check_hip(hipMemsetAsync(h->blob, 0, h->L.total, st), "hipMemsetAsync(blob)");
    if (rc) return rc;
    const int blk = 256;
    const BlobLayout L = h->L;
    if (Na > 0)
        hipLaunchKernelGGL(pack_near_kernel, dim3(grid_for((int64_t)B * Hkv * L.Na_pad * (D / 16), blk)), dim3(blk),
                           0, st, near_k, near_v, near_dtype, L, h->blob);
    hipLaunchKernelGGL(pack_valid_kernel, dim3(grid_for(Hkv, blk)), dim3(blk), 0, st, near_valid, Hkv, L, h->blob);
    hipLaunchKernelGGL(fill_kscale_kernel, dim3(grid_for((int64_t)B * Hkv, blk)), dim3(blk), 0, st, nullptr, B * Hkv,
                       L, h->blob, nullptr);
    return check_hip(hipGetLastError(), "pack kernels");
}

int attn_finish(fkv_attn_impl* h, hipStream_t st) {
    if (int rc = xcd_rule(h->device, st, &h->xcd_mod)) return rc;
    if (env_int("FKV_XCD_LOCAL", 1) == 0) h->xcd_mod = 0;  // read once per handle, at creation
    std::vector<uint32_t> nv_h(h->L.Hkv, 0);
    int rc = check_hip(hipMemcpyAsync(nv_h.data(), h->blob + h->L.near_valid, h->L.Hkv * sizeof(uint32_t),
                                      hipMemcpyDeviceToHost, st), "hipMemcpyAsync(near_valid)");
    if (!rc) rc = check_hip(hipStreamSynchronize(st), "hipStreamSynchronize");
    if (rc) return rc;
    uint32_t mx = 0;
    for (uint32_t v : nv_h) mx = v > mx ? v : mx;
    h->near_plan = (int)cdiv(mx, kTile);
    return FKV_OK;
}

}  // namespace fkv

namespace {

// fp8 K far tier with per-token (fmt 0) or group-32 (fmt 2) INT4 V.
int create_fp8(const char* fn, int fmt, fkv_attn** out, int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F,
               const void* near_k, const void* near_v, int32_t near_dtype, const uint8_t* far_k,
               const uint8_t* far_v, const void* far_v_scale, const void* far_v_zero, int32_t sz_dtype,
               const int32_t* near_valid, float spike_margin, void* stream) {
    const std::string name(fn);
    if (!out) return set_error(name + ": out is NULL");
    *out = nullptr;
    if (B <= 0 || Hkv <= 0 || Na < 0 || F < 0)
        return set_error(name + ": bad shape B=" + std::to_string(B) + " Hkv=" + std::to_string(Hkv) +
                         " Na=" + std::to_string(Na) + " F=" + std::to_string(F));
    if (D != 64 && D != 128) return set_error(name + ": head dim must be 64 or 128, got " + std::to_string(D));
    if (near_dtype < FKV_F16 || near_dtype > FKV_F32 || sz_dtype < FKV_F16 || sz_dtype > FKV_F32)
        return set_error(name + ": unsupported dtype");
    if ((Na > 0 && (!near_k || !near_v)) || (F > 0 && (!far_k || !far_v || !far_v_scale || !far_v_zero)) ||
        !near_valid)
        return set_error(name + ": NULL tier array");
    hipStream_t st = (hipStream_t)stream;
    fkv_attn* h = new fkv_attn();
    unsigned* bad = nullptr;
    int rc = fkv::attn_begin(h, B, Hkv, D, Na, F, fmt, near_k, near_v, near_dtype, near_valid, spike_margin, st);
    if (!rc) rc = check_hip(hipMalloc(&bad, sizeof(unsigned)), "hipMalloc(flag)");
    if (!rc) rc = check_hip(hipMemsetAsync(bad, 0, sizeof(unsigned), st), "hipMemsetAsync");
    if (!rc && F > 0) {
        const int blk = 256;
        const fkv::BlobLayout L = h->L;
        hipLaunchKernelGGL(fkv::pack_far_k_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * L.F_pad * (D / 16), blk)),
                           dim3(blk), 0, st, far_k, L, h->blob, bad);
        if (fmt == 2)
            hipLaunchKernelGGL(fkv::pack_far_v_g32_kernel,
                               dim3(fkv::grid_for((int64_t)B * Hkv * L.F_pad * (D / 8), blk)), dim3(blk), 0, st,
                               far_v, far_v_scale, far_v_zero, sz_dtype, L, h->blob);
        else
            hipLaunchKernelGGL(fkv::pack_far_v_kernel,
                               dim3(fkv::grid_for((int64_t)B * Hkv * L.F_pad * (D / 8), blk)), dim3(blk), 0, st,
                               far_v, far_v_scale, far_v_zero, sz_dtype, L, h->blob);
        rc = check_hip(hipGetLastError(), "far pack kernels");
    }
    unsigned bad_h = 0;
    if (!rc) rc = check_hip(hipMemcpyAsync(&bad_h, bad, sizeof(unsigned), hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    if (!rc) rc = fkv::attn_finish(h, st);
    if (bad) (void)hipFree(bad);
    if (!rc && bad_h) {
        set_error(name + ": far_k holds E4M3 NaN codes 0x7F/0xFF, which the reference encoder never emits");
        rc = FKV_EDATA;
    }
    if (rc) {
        fkv_attn_destroy(h);
        return rc;
    }
    *out = h;
    return FKV_OK;
}

}  // namespace

extern "C" {

int fkv_attn_create(fkv_attn** out, int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F,
                    const void* near_k, const void* near_v, int32_t near_dtype,
                    const uint8_t* far_k, const uint8_t* far_v, const void* far_v_scale,
                    const void* far_v_zero, int32_t sz_dtype, const int32_t* near_valid,
                    float spike_margin, void* stream) {
    return create_fp8("fkv_attn_create", 0, out, B, Hkv, D, Na, F, near_k, near_v, near_dtype, far_k, far_v,
                      far_v_scale, far_v_zero, sz_dtype, near_valid, spike_margin, stream);
}

int fkv_attn_create_g32(fkv_attn** out, int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F,
                        const void* near_k, const void* near_v, int32_t near_dtype,
                        const uint8_t* far_k, const uint8_t* far_v, const void* far_v_scale,
                        const void* far_v_zero, int32_t sz_dtype, const int32_t* near_valid,
                        float spike_margin, void* stream) {
    return create_fp8("fkv_attn_create_g32", 2, out, B, Hkv, D, Na, F, near_k, near_v, near_dtype, far_k, far_v,
                      far_v_scale, far_v_zero, sz_dtype, near_valid, spike_margin, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Scratch of fkv_attn_call_noalloc: the call workspace in a fixed device
// array instead of memory the library allocates.  Layout: [arrival counters
// | fp16 query copy | split partial records]; the counter region has a
// fixed size and place, is zeroed once per device and stays zero between
// calls (the last split of a row re-arms its counter).  Every call on a
// device shares that device's copy: calls that overlap on one device race.
// ---------------------------------------------------------------------------

constexpr size_t kScratchBytes = (size_t)8 << 20;
constexpr int kScratchRows = 16384;  // rows the counter region serves
// arrival counters [rows], then the XCD watch words [1 + rows]
constexpr size_t kScratchArriveBytes = ((size_t)(2 * kScratchRows + 1) * 4 + 255) & ~(size_t)255;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};  // device address of `scratch`, per device

// The current device's address of `scratch` (looked up once per device,
// when its counter region is also cleared, stream-ordered before the call).
int scratch_base(const std::string& name, int dev, hipStream_t st, uint8_t** out) {
    if (dev < 0 || dev >= kScratchDevices) return set_error(name + ": device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        if (int rc = check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
            return rc;
        if (!ptr) return set_error(name + ": hipGetSymbolAddress(scratch) returned NULL");
        const int n = (int)(kScratchArriveBytes / sizeof(int));
        hipLaunchKernelGGL(fkv::zero_ints_kernel, dim3(fkv::grid_for(n, 256)), dim3(256), 0, st, (int*)ptr, n);
        if (int rc = check_hip(hipGetLastError(), "zero_ints_kernel launch")) return rc;
        g_scratch_ptr[dev] = ptr;
    }
    *out = (uint8_t*)g_scratch_ptr[dev];
    return FKV_OK;
}

}  // namespace

namespace {

void free_spike_buffers(fkv_attn* h) {
    void* bufs[] = {h->spk_tmax, h->spk_thr, h->spk_flags, h->spk_tokens, h->spk_cand_n, h->spk_arrive, h->spk_cand_s,
                    h->spk_cand_t};
    for (void* p : bufs)
        if (p) (void)hipFree(p);
    h->spk_tmax = h->spk_thr = h->spk_cand_s = nullptr;
    h->spk_flags = h->spk_tokens = nullptr;
    h->spk_cand_n = h->spk_arrive = h->spk_cand_t = nullptr;
}

// The top-K spike selection's buffers for Hq query heads (spike_k > 1).
int ensure_spike_buffers(fkv_attn* h, int Hq) {
    if (h->spike_k <= 1 || h->spk_hq == Hq) return FKV_OK;
    if (h->spk_hq != 0) return set_error("fkv_attn: spike buffers sized for another query-head count");
    const fkv::BlobLayout& L = h->L;
    const size_t heads = (size_t)L.B * Hq, ntf = (size_t)fkv::cdiv(L.F, fkv::kTile);
    // candidate buffers sized for the largest spike_k, so a later
    // fkv_attn_set_spike_k needs no new allocation
    const size_t cap = (size_t)fkv::kTile * FKV_MAX_SPIKE_K;
    int rc = check_hip(hipMalloc(&h->spk_tmax, (heads * ntf > 0 ? heads * ntf : 1) * sizeof(float)), "hipMalloc(tmax)");
    if (!rc) rc = check_hip(hipMalloc(&h->spk_thr, heads * sizeof(float)), "hipMalloc(thr)");
    if (!rc) rc = check_hip(hipMalloc(&h->spk_flags, heads * sizeof(int32_t)), "hipMalloc(flags)");
    if (!rc) rc = check_hip(hipMalloc(&h->spk_tokens, heads * sizeof(int32_t)), "hipMalloc(tokens)");
    if (!rc) rc = check_hip(hipMalloc(&h->spk_cand_n, heads * sizeof(int)), "hipMalloc(cand_n)");
    // arrival counters of the (batch, KV head, head quad) rows: at most one per query head
    if (!rc) rc = check_hip(hipMalloc(&h->spk_arrive, heads * sizeof(int)), "hipMalloc(arrive)");
    if (!rc) rc = check_hip(hipMalloc(&h->spk_cand_s, heads * cap * sizeof(float)), "hipMalloc(cand_s)");
    if (!rc) rc = check_hip(hipMalloc(&h->spk_cand_t, heads * cap * sizeof(int)), "hipMalloc(cand_t)");
    if (!rc) rc = check_hip(hipMemset(h->spk_cand_n, 0, heads * sizeof(int)), "hipMemset(cand_n)");
    if (!rc) rc = check_hip(hipMemset(h->spk_arrive, 0, heads * sizeof(int)), "hipMemset(arrive)");
    if (rc) {
        free_spike_buffers(h);
        return rc;
    }
    h->spk_hq = Hq;
    return FKV_OK;
}

// The handle's call workspace, allocated by its first call (sized for every
// launch plan of that query-head count) and never re-allocated afterwards.
int ensure_workspace(const std::string& name, fkv_attn* h, int Hq, hipStream_t st) {
    if (h->ws_hq == Hq) return ensure_spike_buffers(h, Hq);
    if (h->ws_hq != 0)
        return set_error(name + ": this handle's workspace was sized by its first call for Hq=" +
                         std::to_string(h->ws_hq) + "; a call with Hq=" + std::to_string(Hq) +
                         " needs a handle of its own");
    const fkv::BlobLayout& L = h->L;
    const size_t wsf = fkv::workspace_floats(L, Hq);
    const int rows = fkv::workspace_rows(L, Hq);
    const size_t qn = (size_t)L.B * Hq * L.D;
    int rc = check_hip(hipMalloc(&h->ws, wsf * sizeof(float)), "hipMalloc(ws)");
    // arrival counters [rows], then the XCD watch words [1 + rows]
    if (!rc) rc = check_hip(hipMalloc(&h->arrive, (2 * (size_t)rows + 1) * sizeof(int)), "hipMalloc(arrive)");
    if (!rc) rc = check_hip(hipMalloc(&h->qbuf, qn * 2), "hipMalloc(qbuf)");
    if (rc) {
        if (h->ws) (void)hipFree(h->ws);
        if (h->arrive) (void)hipFree(h->arrive);
        if (h->qbuf) (void)hipFree(h->qbuf);
        h->ws = nullptr;
        h->arrive = nullptr;
        h->qbuf = nullptr;
        return rc;
    }
    h->ws_floats = wsf;
    h->arrive_n = rows;
    h->ws_hq = Hq;
    if (int rc2 = ensure_spike_buffers(h, Hq)) return rc2;
    // counters and watch words start at zero; the kernel's last split
    // re-arms its row's counter and clears its watch word
    hipLaunchKernelGGL(fkv::zero_ints_kernel, dim3(fkv::grid_for(2 * rows + 1, 256)), dim3(256), 0, st, h->arrive,
                       2 * rows + 1);
    return check_hip(hipGetLastError(), "zero_ints_kernel launch");
}

// n_decode: valid decode rows (host count) or, with n_dec_dev, ignored (the
// kernel reads the count there); dec_stride: rows per (batch, kv head)
// block of decode_k / decode_v.
// The buffers one call's kernels use besides inputs and outputs.
struct CallWorkspace {
    float* ws;           // split partial records
    int* arrive;         // per-row arrival counters, zero between calls
    uint32_t* watch;     // XCD watch words: [0] violations, [1 + row]
    uint16_t* qbuf;      // fp16 copy of a bf16 / f32 query
    size_t ws_floats, arrive_n, qbuf_n;
};

// Lays a call's workspace out in the no-alloc entry point's scratch array
// (below); NULL when the call does not fit.
int scratch_workspace(const std::string& name, fkv_attn* h, const fkv::LaunchPlan& p, int Hq, hipStream_t st,
                      CallWorkspace* out);

int attn_call(const char* fn, fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq, const void* decode_k,
              const void* decode_v, int32_t n_decode, int32_t dec_stride, const int32_t* n_dec_dev, void* out,
              int32_t* spike_flags, int32_t* spike_tokens, void* stream, bool no_alloc = false) {
    const std::string name(fn);
    if (!h || !query || !out || !spike_flags || !spike_tokens) return set_error(name + ": NULL argument");
    const fkv::BlobLayout& L = h->L;
    if (Hq <= 0 || Hq % L.Hkv != 0)
        return set_error(name + ": Hq=" + std::to_string(Hq) + " is not a multiple of H_kv=" + std::to_string(L.Hkv));
    if (n_decode < 0 || dec_stride < n_decode || (dec_stride > 0 && (!decode_k || !decode_v)))
        return set_error(name + ": bad decode buffer");
    if (q_dtype < FKV_F16 || q_dtype > FKV_F32) return set_error(name + ": unsupported query dtype");
    if (q_dtype == FKV_F16 && ((uintptr_t)query & 7) != 0)
        return set_error(name + ": an fp16 query must be 8-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    // order this call after the handle's last eager call when that ran on
    // another stream (fkv_attn_impl::order_ev)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (int rc = check_hip(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing")) return rc;
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (!capturing && h->order_pending && h->order_st != st)
        if (int rc = check_hip(hipStreamWaitEvent(st, h->order_ev, 0), "hipStreamWaitEvent(order)")) return rc;
    const int G = Hq / L.Hkv;
    const bool topk = h->spike_k > 1;
    if (topk && no_alloc && h->spk_hq != Hq)
        return set_error(name + ": spike_k > 1 needs the selection buffers of a call with Hq=" + std::to_string(Hq) +
                         " (fkv_attn_call once, or fkv_attn_set_spike_k after one)");
    // the split count follows the longest decode length the call can see
    const fkv::LaunchPlan p = fkv::plan_launch(L, Hq, n_dec_dev ? dec_stride : n_decode, h->target_wgs);
    CallWorkspace w;
    if (no_alloc) {
        if (int rc = scratch_workspace(name, h, p, Hq, st, &w)) return rc;
    } else {
        if (int rc = ensure_workspace(name, h, Hq, st)) return rc;
        w = CallWorkspace{h->ws, h->arrive, (uint32_t*)(h->arrive + h->arrive_n), h->qbuf, h->ws_floats,
                          h->arrive_n, (size_t)L.B * Hq * L.D};
    }
    if (p.ws_floats > w.ws_floats || p.rows > (int)w.arrive_n)
        return set_error(name + ": launch plan exceeds the workspace (internal error)");
    const int hpg = p.hpg, head_groups = p.head_groups, ng_max = p.ng_max, rows = p.rows, splits = p.splits;
    const uint16_t* q16 = (const uint16_t*)query;
    const int64_t qn = (int64_t)L.B * Hq * L.D;
    if (q_dtype != FKV_F16) {
        if ((size_t)qn > w.qbuf_n) return set_error(name + ": query exceeds the workspace (internal error)");
        hipLaunchKernelGGL(fkv::cast_to_f16_kernel, dim3(fkv::grid_for(qn, 256)), dim3(256), 0, st, query,
                           q_dtype, qn, w.qbuf);
        q16 = w.qbuf;
    }
    fkv::AttnArgs a;
    a.blob = h->blob;
    a.L = L;
    a.q = q16;
    a.dec_k = (const uint16_t*)decode_k;
    a.dec_v = (const uint16_t*)decode_v;
    a.n_dec = n_dec_dev ? 0 : n_decode;
    a.dec_stride = dec_stride;
    a.n_dec_dev = n_dec_dev;
    a.Hq = Hq;
    a.G = G;
    a.head_groups = head_groups;
    a.hpg = hpg;
    a.num_splits = splits;
    a.wave_recs = p.wave_recs;
    // the XCD-local merge needs whole XCD groups of rows (the grid's rows,
    // Hkv * head_groups * B, are p.rows)
    a.xcd_mod = h->xcd_mod > 0 && splits > 1 && h->fused_merge && rows % h->xcd_mod == 0 ? h->xcd_mod : 0;
    a.spike_margin = h->margin;
    a.inv_sqrt_d = (float)(1.0 / sqrt((double)L.D));
    a.out = (uint16_t*)out;
    // spike_k > 1: the attention kernel's flag / argmax, tile maxima and
    // thresholds go to the selection's buffers; the selection writes
    // the caller's spike outputs
    a.flags = topk ? h->spk_flags : spike_flags;
    a.tokens = topk ? h->spk_tokens : spike_tokens;
    a.tmax = topk ? h->spk_tmax : nullptr;
    a.tmax_stride = (int)fkv::cdiv(L.F, fkv::kTile);
    a.thr = topk ? h->spk_thr : nullptr;
    a.kscale = h->has_kscale ? (const float*)(h->blob + L.kscale) : nullptr;
#ifdef FKV_PHASE_STAMPS
    {
        void* sp = nullptr;
        if (int rc = check_hip(hipGetSymbolAddress(&sp, HIP_SYMBOL(fkv::fkv_stamps)), "hipGetSymbolAddress(stamps)"))
            return rc;
        a.stamps = (unsigned long long*)sp;
    }
#endif
    a.ws = w.ws;
    const bool fused_merge = h->fused_merge;
    a.arrive = fused_merge ? w.arrive : nullptr;
    a.xcd_watch = w.watch;
    a.near_plan = h->near_plan;
    {
        // Decode tiles go to the wave with the fewest planned bytes where a
        // wave's far share is below one near tile (the near tiles then
        // decide the balance): after the near tiles when far tiles are dealt
        // round-robin.  Where the far split is byte-balanced over many far
        // tiles, from wave 0 (the waves without near tiles hold their share
        // in far tiles, slower per byte).
        const int nw = splits * p.waves, FT = (int)fkv::cdiv(L.F, fkv::kTile);
        const int64_t NB = fkv::near_tile_weight((ng_max + 3) / 4, L.D), FB = (int64_t)L.far_rec;
        a.dec_wave0 = 0;
        if ((int64_t)FT * FB < nw * NB) {
            if (fkv::far_round_robin(L.fmt == 1, nw, FT, NB, FB)) {
                a.dec_wave0 = (fkv::near_deal_start(true, nw, FT, NB, FB) + h->near_plan) % nw;
            } else {
                int64_t best = -1;
                for (int w = 0; w < nw; w++) {
                    const int64_t nn = h->near_plan / nw + (w < h->near_plan % nw ? 1 : 0);
                    const int64_t nf = fkv::far_bound(w + 1, nw, h->near_plan, FT, NB, FB) -
                                       fkv::far_bound(w, nw, h->near_plan, FT, NB, FB);
                    const int64_t cost = nn * NB + nf * FB;
                    if (best < 0 || cost < best) {
                        best = cost;
                        a.dec_wave0 = w;
                    }
                }
            }
        }
    }
    const dim3 grid(splits, L.Hkv * head_groups, L.B), block(fkv::kWave * p.waves);
    a.tq_rot = h->tq.rot;
    a.tq_alpha = h->tq.alpha;
    a.tq_beta = h->tq.beta;
    a.tq_gamma = h->tq.gamma;
    a.tq_delta = h->tq.delta;
    a.tq_qjl = 1.2533141f / (float)L.D;
    a.tq_lvh = h->tq.lvh;
    a.tq_lvl = h->tq.lvl;
    const int nq = (ng_max + 3) / 4;
    const bool ext = topk || h->has_kscale;  // the kernels that carry the extensions
    fkv::AttnKernel k = L.fmt == 1 ? (L.D == 128 ? fkv::pick_attn_turbo<128>(nq) : fkv::pick_attn_turbo<64>(nq))
                        : nq == 1  ? fkv::attn_kernel_one_quad(L.D, L.fmt, ext, topk)
                                   : fkv::attn_kernel_quads(L.D, L.fmt, nq, ext, topk);
    hipLaunchKernelGGL(k, grid, block, 0, st, a);
    if (splits > 1 && !fused_merge) {
        const dim3 mgrid(rows, ng_max);
        if (L.D == 128) hipLaunchKernelGGL(fkv::merge_kernel<128>, mgrid, dim3(fkv::kWave), 0, st, a);
        else hipLaunchKernelGGL(fkv::merge_kernel<64>, mgrid, dim3(fkv::kWave), 0, st, a);
    }
    if (topk) {
        fkv::SelectArgs sa;
        sa.blob = h->blob;
        sa.L = L;
        sa.q = q16;
        sa.Hq = Hq;
        sa.G = G;
        sa.K = h->spike_k;
        sa.inv_sqrt_d = a.inv_sqrt_d;
        sa.tmax = h->spk_tmax;
        sa.ntf = a.tmax_stride;
        sa.thr = h->spk_thr;
        sa.flags_in = h->spk_flags;
        sa.tokens_in = h->spk_tokens;
        sa.flags = spike_flags;
        sa.tokens = spike_tokens;
        sa.kscale = a.kscale;
        sa.cand_n = h->spk_cand_n;
        sa.arrive = h->spk_arrive;
        sa.cand_s = h->spk_cand_s;
        sa.cand_t = h->spk_cand_t;
        sa.cap = fkv::kTile * h->spike_k;
#ifdef FKV_PHASE_STAMPS
        sa.stamps = a.stamps;
#endif
        const unsigned quads = (unsigned)fkv::cdiv(G, 4);
        const dim3 cgrid(quads * fkv::kSelParts, L.Hkv, L.B);
        const dim3 sblock(fkv::kWave * fkv::kSelWaves);
        if (L.D == 128) hipLaunchKernelGGL(fkv::spike_candidates_kernel<128>, cgrid, sblock, 0, st, sa);
        else hipLaunchKernelGGL(fkv::spike_candidates_kernel<64>, cgrid, sblock, 0, st, sa);
    }
    if (int rc = check_hip(hipGetLastError(), "attn_kernel launch")) return rc;
    if (capturing) return FKV_OK;
    if (!h->order_ev)
        if (int rc = check_hip(hipEventCreateWithFlags(&h->order_ev, hipEventDisableTiming), "hipEventCreate(order)"))
            return rc;
    if (int rc = check_hip(hipEventRecord(h->order_ev, st), "hipEventRecord(order)")) return rc;
    h->order_st = st;
    h->order_pending = true;
    return FKV_OK;
}

int scratch_workspace(const std::string& name, fkv_attn* h, const fkv::LaunchPlan& p, int Hq, hipStream_t st,
                      CallWorkspace* out) {
    const fkv::BlobLayout& L = h->L;
    const size_t qbytes = ((size_t)L.B * Hq * L.D * 2 + 255) & ~(size_t)255;
    const size_t need = kScratchArriveBytes + qbytes + p.ws_floats * sizeof(float);
    if (p.rows > kScratchRows || need > kScratchBytes)
        return set_error(name + ": this call needs " + std::to_string(need) + " bytes of scratch (" +
                         std::to_string(p.rows) + " rows x " + std::to_string(p.splits) +
                         " splits); the no-alloc entry point holds " + std::to_string(kScratchBytes) +
                         " bytes -- use fkv_attn_call");
    int dev = -1;
    if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev != h->device) return set_error(name + ": the handle's device must be current");
    uint8_t* base = nullptr;
    if (int rc = scratch_base(name, dev, st, &base)) return rc;
    out->arrive = (int*)base;
    out->arrive_n = kScratchRows;
    out->watch = (uint32_t*)(base + (size_t)kScratchRows * sizeof(int));
    out->qbuf = (uint16_t*)(base + kScratchArriveBytes);
    out->qbuf_n = qbytes / 2;
    out->ws = (float*)(base + kScratchArriveBytes + qbytes);
    out->ws_floats = (kScratchBytes - kScratchArriveBytes - qbytes) / sizeof(float);
    return FKV_OK;
}

}  // namespace

extern "C" {

int fkv_attn_call(fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq,
                  const void* decode_k, const void* decode_v, int32_t n_decode, void* out,
                  int32_t* spike_flags, int32_t* spike_tokens, void* stream) {
    return attn_call("fkv_attn_call", h, query, q_dtype, Hq, decode_k, decode_v, n_decode, n_decode, nullptr, out,
                     spike_flags, spike_tokens, stream);
}

int fkv_attn_call_strided(fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq, const void* decode_k,
                          const void* decode_v, int32_t n_decode, int32_t row_stride, void* out,
                          int32_t* spike_flags, int32_t* spike_tokens, void* stream) {
    return attn_call("fkv_attn_call_strided", h, query, q_dtype, Hq, decode_k, decode_v, n_decode, row_stride,
                     nullptr, out, spike_flags, spike_tokens, stream);
}

int fkv_attn_call_noalloc(fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq, const void* decode_k,
                          const void* decode_v, int32_t n_decode, void* out, int32_t* spike_flags,
                          int32_t* spike_tokens, void* stream) {
    return attn_call("fkv_attn_call_noalloc", h, query, q_dtype, Hq, decode_k, decode_v, n_decode, n_decode,
                     nullptr, out, spike_flags, spike_tokens, stream, true);
}

int fkv_attn_plan(int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F, int32_t Hq, int32_t n_decode,
                  int32_t target_wgs, int32_t fmt, int64_t* out) {
    if (B <= 0 || Hkv <= 0 || (D != 64 && D != 128) || Na < 0 || F < 0 || Hq <= 0 || Hq % Hkv != 0 ||
        n_decode < 0 || target_wgs < 1 || fmt < 0 || fmt > 2 || !out)
        return set_error("fkv_attn_plan: bad argument");
    const fkv::BlobLayout L = fkv::make_layout(B, Hkv, D, Na, F, fmt);
    const fkv::LaunchPlan p = fkv::plan_launch(L, Hq, n_decode, target_wgs);
    out[0] = p.hpg;
    out[1] = p.rows;
    out[2] = p.splits;
    out[3] = (int64_t)p.ws_floats;
    out[4] = (int64_t)fkv::workspace_floats(L, Hq);
    out[5] = fkv::workspace_rows(L, Hq);
    out[6] = p.waves;
    out[7] = p.wave_recs;
    return FKV_OK;
}

int fkv_far_plan(int32_t n_waves, int32_t near_plan, int32_t nt_far, int64_t near_weight, int64_t far_rec,
                 int32_t turbo, int32_t* f0, int32_t* fs, int32_t* nf) {
    if (n_waves <= 0 || near_plan < 0 || nt_far < 0 || near_weight <= 0 || far_rec <= 0 || !f0 || !fs || !nf)
        return set_error("fkv_far_plan: bad argument");
    for (int w = 0; w < n_waves; w++) {
        const fkv::FarPlan p = fkv::plan_far(w, n_waves, nt_far, near_plan, far_rec, turbo != 0, near_weight);
        f0[w] = p.f0;
        fs[w] = p.fs;
        nf[w] = p.nf;
    }
    return FKV_OK;
}

int fkv_attn_call_dev(fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq, const void* decode_k,
                      const void* decode_v, const int32_t* n_decode_dev, int32_t capacity, void* out,
                      int32_t* spike_flags, int32_t* spike_tokens, void* stream) {
    if (!n_decode_dev) return set_error("fkv_attn_call_dev: NULL n_decode_dev");
    return attn_call("fkv_attn_call_dev", h, query, q_dtype, Hq, decode_k, decode_v, capacity, capacity,
                     n_decode_dev, out, spike_flags, spike_tokens, stream);
}

int fkv_e4m3_decode(const uint8_t* codes, void* out_f16, int64_t n, void* stream) {
    if (n < 0 || n % 4 != 0 || (n > 0 && (!codes || !out_f16)))
        return set_error("fkv_e4m3_decode: n must be a multiple of 4 with non-NULL buffers");
    if (n == 0) return FKV_OK;
    hipLaunchKernelGGL(fkv::e4m3_decode_kernel, dim3(fkv::grid_for(n / 4, 256)), dim3(256), 0,
                       (hipStream_t)stream, codes, (uint16_t*)out_f16, n / 4);
    return check_hip(hipGetLastError(), "e4m3_decode_kernel launch");
}

int fkv_attn_dispatch_info(const fkv_attn* h, int32_t* xcd_mod) {
    if (!h || !xcd_mod) return set_error("fkv_attn_dispatch_info: NULL argument");
    *xcd_mod = h->xcd_mod;
    return FKV_OK;
}

int fkv_phase_stamps(uint64_t* out, int32_t n_wgs, int32_t clear) {
#ifdef FKV_PHASE_STAMPS
    if (n_wgs < 0 || n_wgs > fkv::kStampWGs || (n_wgs > 0 && !out)) return set_error("fkv_phase_stamps: bad argument");
    const size_t bytes = sizeof(uint64_t) * fkv::kStampSlots * (size_t)n_wgs;
    if (n_wgs > 0) {
        if (int rc = check_hip(hipMemcpyFromSymbol(out, HIP_SYMBOL(fkv::fkv_stamps), bytes, 0, hipMemcpyDeviceToHost),
                               "hipMemcpyFromSymbol(stamps)"))
            return rc;
    }
    if (clear) {
        std::vector<uint64_t> z((size_t)fkv::kStampSlots * fkv::kStampWGs, 0);
        if (int rc = check_hip(hipMemcpyToSymbol(HIP_SYMBOL(fkv::fkv_stamps), z.data(), z.size() * 8, 0,
                                                 hipMemcpyHostToDevice),
                               "hipMemcpyToSymbol(stamps)"))
            return rc;
    }
    return FKV_OK;
#else
    (void)out;
    (void)n_wgs;
    (void)clear;
    return set_error("fkv_phase_stamps: this library was built without FKV_PHASE_STAMPS");
#endif
}

int fkv_xcd_rule_fit(const uint32_t* xcc, int32_t n, int32_t* xcd_mod, int32_t* offset) {
    if (!xcc || n <= 0 || !xcd_mod || !offset) return set_error("fkv_xcd_rule_fit: bad argument");
    uint32_t lo = xcc[0], hi = xcc[0];
    for (int32_t i = 0; i < n; i++) {
        lo = xcc[i] < lo ? xcc[i] : lo;
        hi = xcc[i] > hi ? xcc[i] : hi;
    }
    const uint32_t X = hi - lo + 1, c = xcc[0] - lo;
    bool ok = X <= 32;
    for (int32_t i = 0; i < n && ok; i++) ok = xcc[i] == lo + (c + (uint32_t)i) % X;
    *xcd_mod = ok ? (int32_t)X : 0;
    *offset = ok ? (int32_t)c : 0;
    return FKV_OK;
}

int32_t fkv_xcd_watch_violations(const uint32_t* words, int32_t rows) {
    if (!words || rows < 0) return set_error("fkv_xcd_watch_violations: bad argument");
    int32_t v = words[0] != 0;
    for (int32_t r = 0; r < rows; r++) v += words[1 + r] != 0;  // arrival counters left armed
    return v;
}

int fkv_attn_dispatch_check(fkv_attn* h, int32_t* violations, void* stream) {
    if (!h || !violations) return set_error("fkv_attn_dispatch_check: NULL argument");
    *violations = 0;
    hipStream_t st = (hipStream_t)stream;
    if (int rc = check_hip(hipStreamSynchronize(st), "hipStreamSynchronize")) return rc;
    // the handle's own watch words, and the device's no-alloc scratch words
    struct Region {
        int* arrive;
        int rows;
    };
    std::vector<Region> regions;
    if (h->arrive) regions.push_back({h->arrive, (int)h->arrive_n});
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (h->device >= 0 && h->device < kScratchDevices && g_scratch_ptr[h->device])
            regions.push_back({(int*)g_scratch_ptr[h->device], kScratchRows});
    }
    int32_t total = 0;
    for (const Region& r : regions) {
        // [flag, counters of rows 0..rows-1]: at rest every counter is zero
        // (each row's merging workgroup re-arms it)
        std::vector<uint32_t> w((size_t)r.rows + 1);
        int rc = check_hip(hipMemcpyAsync(w.data(), r.arrive + r.rows, 4, hipMemcpyDeviceToHost, st),
                           "hipMemcpyAsync(xcd watch)");
        if (!rc) rc = check_hip(hipMemcpyAsync(w.data() + 1, r.arrive, (size_t)r.rows * 4, hipMemcpyDeviceToHost, st),
                                "hipMemcpyAsync(arrival counters)");
        if (!rc) rc = check_hip(hipStreamSynchronize(st), "hipStreamSynchronize");
        if (rc) return rc;
        const int32_t v = fkv_xcd_watch_violations(w.data(), r.rows);
        if (v > 0) {
            // the arrival counts of the broken dispatches were split across
            // L2s: clear counters and watch words before the coherent merge
            hipLaunchKernelGGL(fkv::zero_ints_kernel, dim3(fkv::grid_for(2 * r.rows + 1, 256)), dim3(256), 0, st,
                               r.arrive, 2 * r.rows + 1);
            if (int rc = check_hip(hipGetLastError(), "zero_ints_kernel launch")) return rc;
        }
        total += v;
    }
    if (total > 0) h->xcd_mod = 0;  // later calls merge through memory
    *violations = total;
    return FKV_OK;
}

int fkv_attn_blob_info(const fkv_attn* h, fkv_blob_info* out) {
    if (!h || !out) return set_error("fkv_attn_blob_info: NULL argument");
    out->blob = h->blob;
    out->blob_bytes = h->L.total;
    out->near_k_offset = h->L.near_k;
    out->near_v_offset = h->L.near_v;
    out->near_valid_offset = h->L.near_valid;
    out->n_near_alloc = h->L.Na;
    out->n_far = h->L.F;
    out->B = h->L.B;
    out->H_kv = h->L.Hkv;
    out->D = h->L.D;
    return FKV_OK;
}

int fkv_attn_read_near_valid(const fkv_attn* h, uint32_t* host_out, void* stream) {
    if (!h || !host_out) return set_error("fkv_attn_read_near_valid: NULL argument");
    hipStream_t st = (hipStream_t)stream;
    int rc = check_hip(hipMemcpyAsync(host_out, h->blob + h->L.near_valid, h->L.Hkv * sizeof(uint32_t),
                                      hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    if (!rc) rc = check_hip(hipStreamSynchronize(st), "hipStreamSynchronize");
    return rc;
}

int fkv_attn_promote_rows(fkv_attn* h, int32_t n, const int32_t* head_slot, const void* rows_k,
                          const void* rows_v, int32_t row_batches, void* stream) {
    if (!h || n < 0 || (n > 0 && (!head_slot || !rows_k || !rows_v)))
        return set_error("fkv_attn_promote_rows: NULL argument or negative count");
    if (row_batches < 1 || row_batches > h->L.B)
        return set_error("fkv_attn_promote_rows: row_batches must be in [1, B]");
    if (n == 0) return FKV_OK;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(fkv::promote_rows_kernel, dim3(n), dim3(256), 0, st, head_slot, (const uint16_t*)rows_k,
                       (const uint16_t*)rows_v, n, row_batches, h->L, h->blob);
    hipLaunchKernelGGL(fkv::bump_near_valid_kernel, dim3(1), dim3(256), 0, st, head_slot, n, h->L, h->blob);
    return check_hip(hipGetLastError(), "promote kernels launch");
}

int fkv_attn_export_near(const fkv_attn* h, void* near_k_out, void* near_v_out, void* stream) {
    if (!h || (!near_k_out && !near_v_out)) return set_error("fkv_attn_export_near: NULL argument");
    const int64_t n = (int64_t)h->L.B * h->L.Hkv * h->L.Na * h->L.D;
    if (n == 0) return FKV_OK;
    hipLaunchKernelGGL(fkv::export_near_kernel, dim3(fkv::grid_for(n, 256)), dim3(256), 0, (hipStream_t)stream, h->L,
                       h->blob, (uint16_t*)near_k_out, (uint16_t*)near_v_out);
    return check_hip(hipGetLastError(), "export_near_kernel launch");
}

int fkv_attn_set_spike_k(fkv_attn* h, int32_t spike_k) {
    if (!h) return set_error("fkv_attn_set_spike_k: NULL handle");
    if (spike_k < 1 || spike_k > FKV_MAX_SPIKE_K)
        return set_error("fkv_attn_set_spike_k: spike_k must be in [1, " + std::to_string(FKV_MAX_SPIKE_K) + "], got " +
                         std::to_string(spike_k));
    if (spike_k > 1 && h->L.fmt == 1)
        return set_error("fkv_attn_set_spike_k: TurboQuant handles select one spike token per head (spike_k = 1)");
    h->spike_k = spike_k;
    // a handle whose workspace exists gets the selection buffers now, so
    // later calls (and fkv_attn_call_noalloc) allocate nothing
    return h->ws_hq ? ensure_spike_buffers(h, h->ws_hq) : FKV_OK;
}

int fkv_attn_set_k_scale(fkv_attn* h, const float* k_scale, void* stream) {
    if (!h || !k_scale) return set_error("fkv_attn_set_k_scale: NULL argument");
    if (h->L.fmt == 1) return set_error("fkv_attn_set_k_scale: TurboQuant handles have no fp8 keys");
    hipStream_t st = (hipStream_t)stream;
    const int n = h->L.B * h->L.Hkv;
    unsigned* bad = nullptr;
    unsigned bad_h = 0;
    int rc = check_hip(hipMalloc(&bad, sizeof(unsigned)), "hipMalloc(flag)");
    if (!rc) rc = check_hip(hipMemsetAsync(bad, 0, sizeof(unsigned), st), "hipMemsetAsync");
    if (!rc) {
        hipLaunchKernelGGL(fkv::fill_kscale_kernel, dim3(fkv::grid_for(n, 256)), dim3(256), 0, st, k_scale, n, h->L,
                           h->blob, bad);
        rc = check_hip(hipGetLastError(), "fill_kscale_kernel launch");
    }
    if (!rc) rc = check_hip(hipMemcpyAsync(&bad_h, bad, sizeof(unsigned), hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    if (!rc) rc = check_hip(hipStreamSynchronize(st), "hipStreamSynchronize");
    if (bad) (void)hipFree(bad);
    if (!rc && bad_h) {
        set_error("fkv_attn_set_k_scale: a key scale is not a positive finite number");
        return FKV_EDATA;
    }
    if (!rc) h->has_kscale = true;
    return rc;
}

void fkv_attn_destroy(fkv_attn* h) {
    if (!h) return;
    if (h->blob) (void)hipFree(h->blob);
    free_spike_buffers(h);
    if (h->ws) (void)hipFree(h->ws);
    if (h->qbuf) (void)hipFree(h->qbuf);
    if (h->arrive) (void)hipFree(h->arrive);
    if (h->tq.rot) (void)hipFree(h->tq.rot);
    if (h->order_ev) (void)hipEventDestroy(h->order_ev);
    delete h;
}

}  // extern "C"
