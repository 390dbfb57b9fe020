// Fused two-tier split-K decode attention for gfx950 (fp8-E4M3 K / INT4 V far
// tier, fp16 near tier, fp16 decode buffer) and the per-layer device blob.
//
// Replaces the reference's FoveatedHandle + foveated_2tier Metal kernel
// (csrc/foveated_attn.cpp:83-254, csrc/kernels/foveated_attn.metal:181-432).
//
// Work decomposition: one workgroup of 4 waves per (batch, kv_head, split)
// serves every query head of the GQA group, so each compressed byte is read
// from HBM once.  A wave processes 64-token tiles:
//   * scores are token-parallel (lane = token): K is widened to fp16 in
//     registers (E4M3 -> fp16 with the native converter, exact) and dotted
//     with the unscaled fp16 query via v_dot2_f32_f16 (exact products, fp32
//     accumulation); the 1/sqrt(D) scale is applied to the fp32 score;
//   * online softmax per head with one max reduction per tile;
//   * P.V is d-parallel: lane = (phase, 8-dim block), token pairs are packed
//     into half2 and accumulated with v_dot2_f32_f16 into fp32.  INT4 codes
//     are widened exactly to fp16 (16 + c) by bit insertion; the weights are
//     p*scale, the values re-centred to (c - 7.5), and the zero point plus
//     the constant offsets are folded into per-head scalar terms.
// Split partials are merged by a small second kernel (one workgroup per
// (batch, kv_head, head group)).
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstring>
#include <vector>

#include "fkv_common.h"
#include "fkv_attn.h"

namespace fkv {

// ---------------------------------------------------------------------------
// Blob layout
// ---------------------------------------------------------------------------

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

BlobLayout make_layout(int B, int Hkv, int D, int Na, int F) {
    BlobLayout L{};
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
    L.far_k = place(bkv * L.F_pad * D);
    L.far_v = place(bkv * L.F_pad * D / 2);
    L.far_sz = place(bkv * L.F_pad * 4);
    L.near_valid = place((size_t)Hkv * 4);
    L.total = off;
    return L;
}

// ---------------------------------------------------------------------------
// Blob packing kernels (handle construction; csrc/foveated_attn.cpp:83-128)
// ---------------------------------------------------------------------------

__device__ inline uint16_t load_as_f16(const void* p, int64_t i, int dtype) {
    if (dtype == FKV_F16) return ((const uint16_t*)p)[i];
    if (dtype == FKV_BF16) return f2h(bf2f(((const uint16_t*)p)[i]));
    return f2h(((const float*)p)[i]);
}

// near K -> token-parallel tiles: [tile][d/8][lane][8 halves]; near V -> rows.
// One thread per (bkv, token, 8-dim chunk).  Rows >= Na are zero.
__global__ void pack_near_kernel(const void* __restrict__ nk, const void* __restrict__ nv,
                                 int dtype, BlobLayout L, uint8_t* __restrict__ blob) {
    const int D = L.D, C = D / 8;
    const int64_t n = (int64_t)L.B * L.Hkv * L.Na_pad * C;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % C);
        const int64_t r = i / C;
        const int t = (int)(r % L.Na_pad);
        const int64_t bkv = r / L.Na_pad;
        uint16_t kk[8], vv[8];
        for (int e = 0; e < 8; e++) {
            if (t < L.Na) {
                const int64_t src = (bkv * L.Na + t) * D + c * 8 + e;
                kk[e] = load_as_f16(nk, src, dtype);
                vv[e] = load_as_f16(nv, src, dtype);
            } else {
                kk[e] = 0;
                vv[e] = 0;
            }
        }
        uint16_t* kt = (uint16_t*)(blob + L.near_k) +
                       bkv * (int64_t)L.Na_pad * D + (int64_t)(t / kTile) * kTile * D +
                       (int64_t)c * kTile * 8 + (t % kTile) * 8;
        uint16_t* vr = (uint16_t*)(blob + L.near_v) + (bkv * L.Na_pad + t) * D + c * 8;
        for (int e = 0; e < 8; e++) {
            kt[e] = kk[e];
            vr[e] = vv[e];
        }
    }
}

// far K codes -> [tile][d/16][lane][16 codes]; exponent-0 codes are written
// as signed zero (the reference LUT ignores their mantissa); NaN codes are
// reported through *bad.
__global__ void pack_far_k_kernel(const uint8_t* __restrict__ fk, BlobLayout L,
                                  uint8_t* __restrict__ blob, unsigned* __restrict__ bad) {
    const int D = L.D, C = D / 16;
    const int64_t n = (int64_t)L.B * L.Hkv * L.F_pad * C;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % C);
        const int64_t r = i / C;
        const int t = (int)(r % L.F_pad);
        const int64_t bkv = r / L.F_pad;
        uint8_t* dst = blob + L.far_k + bkv * (int64_t)L.F_pad * D + (int64_t)(t / kTile) * kTile * D +
                       (int64_t)c * kTile * 16 + (t % kTile) * 16;
        for (int e = 0; e < 16; e++) {
            uint8_t b = 0;
            if (t < L.F) {
                b = fk[(bkv * L.F + t) * D + c * 16 + e];
                if ((b & 0x7F) == 0x7F) atomicOr(bad, 1u);
                if ((b & 0x78) == 0) b &= 0x80;
            }
            dst[e] = b;
        }
    }
}

// far V nibbles -> per group of GS = 4*NPH tokens: [group][lane=(ph,qb)][4 x 4 bytes]
// where dword i holds dims 8qb..8qb+7 of token ph + NPH*i; scale/zero -> half2.
__global__ void pack_far_v_kernel(const uint8_t* __restrict__ fv, const void* __restrict__ fvs,
                                  const void* __restrict__ fvz, int sz_dtype, BlobLayout L,
                                  uint8_t* __restrict__ blob) {
    const int D = L.D, NQ = D / 8, NPH = kWave / NQ, GS = 4 * NPH;
    const int64_t n = (int64_t)L.B * L.Hkv * L.F_pad * NQ;  // one 4-byte block per thread
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int qb = (int)(i % NQ);
        const int64_t r = i / NQ;
        const int t = (int)(r % L.F_pad);
        const int64_t bkv = r / L.F_pad;
        uint32_t word = 0;
        if (t < L.F) {
            const uint8_t* src = fv + (bkv * L.F + t) * (D / 2) + qb * 4;
            word = (uint32_t)src[0] | ((uint32_t)src[1] << 8) | ((uint32_t)src[2] << 16) |
                   ((uint32_t)src[3] << 24);
        }
        const int j = t / GS, rr = t % GS, ph = rr % NPH, ii = rr / NPH;
        uint32_t* dst = (uint32_t*)(blob + L.far_v + bkv * (int64_t)L.F_pad * D / 2);
        dst[(int64_t)j * (kWave * 4) + (ph * NQ + qb) * 4 + ii] = word;
        if (qb == 0) {
            uint32_t sz = 0;
            if (t < L.F) {
                const int64_t k = bkv * L.F + t;
                sz = (uint32_t)load_as_f16(fvs, k, sz_dtype) |
                     ((uint32_t)load_as_f16(fvz, k, sz_dtype) << 16);
            }
            ((uint32_t*)(blob + L.far_sz))[bkv * L.F_pad + t] = sz;
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

// ---------------------------------------------------------------------------
// Attention kernel
// ---------------------------------------------------------------------------

struct AttnArgs {
    const uint8_t* blob;
    BlobLayout L;
    const uint16_t* q;      // (B, Hq, D) fp16
    const uint16_t* dec_k;  // (B, Hkv, n_dec, D) fp16
    const uint16_t* dec_v;
    int n_dec;
    int Hq;
    int G;          // query heads per kv head
    int head_groups;  // workgroup rows per kv head (G > kMaxG)
    int num_splits;
    float spike_margin;
    float inv_sqrt_d;
    uint16_t* out;  // (B, Hq, D) fp16
    int32_t* flags;
    int32_t* tokens;
    float* ws;          // split partials
};

// Per-head partial record in LDS / workspace: m, l, min_near, max_far, arg, acc[D]
template <int D>
struct Rec {
    static constexpr int kHdr = 5;
    static constexpr int kSize = kHdr + D;
};

template <int D>
__device__ inline void finalize_rows(const AttnArgs& a, const float* fin, int GG_, int b, int head0, int ng);

template <int D, int GG>
struct WaveState {
    float m[GG];
    float lsum[GG];
    float zsum[GG];
    float wsum[GG];  // sum of the fp16-rounded far weights (removes the +16 decode offset)
    float mn[GG];
    float mx[GG];
    int arg[GG];
    float acc[GG][8];
};

// Tile kinds in the virtual sequence [near | far | decode].
enum TileKind { kNear = 0, kFar = 1, kDec = 2 };

template <int D, int GG>
__device__ inline void score_tile(const AttnArgs& a, int kind, int tile, int64_t bkv,
                                  int count, const fkv_h2* __restrict__ qs, float (&s)[GG],
                                  uint32_t& sz) {
    const int lane = threadIdx.x % kWave;
    const int tok = tile * kTile + lane;
    const bool valid = tok < count;
#pragma unroll
    for (int g = 0; g < GG; g++) s[g] = 0.f;
    sz = 0;
    if (kind == kFar) {
        constexpr int C = D / 16;
        const uint4* kt = (const uint4*)(a.blob + a.L.far_k) +
                          (bkv * a.L.F_pad + (int64_t)tile * kTile) * D / 16 + lane;
        uint4 kc[C];
#pragma unroll
        for (int c = 0; c < C; c++) kc[c] = kt[c * kTile];
        sz = ((const uint32_t*)(a.blob + a.L.far_sz))[bkv * a.L.F_pad + tok];
#pragma unroll
        for (int c = 0; c < C; c++) {
            fkv_h2 k2[8];
            k2[0] = e4m3x2_to_h2(kc[c].x, false);
            k2[1] = e4m3x2_to_h2(kc[c].x, true);
            k2[2] = e4m3x2_to_h2(kc[c].y, false);
            k2[3] = e4m3x2_to_h2(kc[c].y, true);
            k2[4] = e4m3x2_to_h2(kc[c].z, false);
            k2[5] = e4m3x2_to_h2(kc[c].z, true);
            k2[6] = e4m3x2_to_h2(kc[c].w, false);
            k2[7] = e4m3x2_to_h2(kc[c].w, true);
#pragma unroll
            for (int g = 0; g < GG; g++) {
                uint4 q0, q1;
                __builtin_memcpy(&q0, qs + g * (D / 2) + c * 8, 16);
                __builtin_memcpy(&q1, qs + g * (D / 2) + c * 8 + 4, 16);
                float acc = s[g];
                acc = dot2(as_h2(q0.x), k2[0], acc);
                acc = dot2(as_h2(q0.y), k2[1], acc);
                acc = dot2(as_h2(q0.z), k2[2], acc);
                acc = dot2(as_h2(q0.w), k2[3], acc);
                acc = dot2(as_h2(q1.x), k2[4], acc);
                acc = dot2(as_h2(q1.y), k2[5], acc);
                acc = dot2(as_h2(q1.z), k2[6], acc);
                acc = dot2(as_h2(q1.w), k2[7], acc);
                s[g] = acc;
            }
        }
    } else {
        constexpr int C = D / 8;
        const uint4* base;
        int64_t stride;  // in uint4 between chunks
        if (kind == kNear) {
            base = (const uint4*)(a.blob + a.L.near_k) +
                   (bkv * a.L.Na_pad + (int64_t)tile * kTile) * D / 8 + lane;
            stride = kTile;
        } else {
            base = (const uint4*)(a.dec_k + (bkv * a.n_dec + (valid ? tok : 0)) * D);
            stride = 1;
        }
        if (valid || kind == kNear) {
#pragma unroll
            for (int half = 0; half < 2; half++) {
                uint4 kc[C / 2];
#pragma unroll
                for (int c = 0; c < C / 2; c++) kc[c] = base[(half * (C / 2) + c) * stride];
#pragma unroll
                for (int c = 0; c < C / 2; c++) {
                    const int cc = half * (C / 2) + c;
#pragma unroll
                    for (int g = 0; g < GG; g++) {
                        uint4 q0;
                        __builtin_memcpy(&q0, qs + g * (D / 2) + cc * 4, 16);
                        float acc = s[g];
                        acc = dot2(as_h2(q0.x), as_h2(kc[c].x), acc);
                        acc = dot2(as_h2(q0.y), as_h2(kc[c].y), acc);
                        acc = dot2(as_h2(q0.z), as_h2(kc[c].z), acc);
                        acc = dot2(as_h2(q0.w), as_h2(kc[c].w), acc);
                        s[g] = acc;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int g = 0; g < GG; g++) s[g] = valid ? s[g] * a.inv_sqrt_d : -INFINITY;
}

// d-parallel P.V over one tile.  pl: this wave's LDS weights [GG][64] (slot order).
template <int D, int GG>
__device__ inline void pv_tile(const AttnArgs& a, int kind, int tile, int64_t bkv, int count,
                               const _Float16* __restrict__ pl, const uint4 (&vfar)[kTile / (4 * (kWave / (D / 8)))],
                               WaveState<D, GG>& st) {
    constexpr int NQ = D / 8, NPH = kWave / NQ, GS = 4 * NPH, NG = kTile / GS;
    const int lane = threadIdx.x % kWave;
    const int ph = lane / NQ, qb = lane % NQ;
#pragma unroll
    for (int j = 0; j < NG; j++) {
        fkv_h2 v01[8], v23[8];
        if (kind == kFar) {
            // nibble c of tokens (A, B) -> half2 (16 + c_A, 16 + c_B): exponent-19
            // fp16 with c in mantissa bits 6..9 (exact); the constant 16 is
            // removed through the per-head weight sum (wsum) at the end.
            const uint4 w = vfar[j];
            uint32_t pr[2][2] = {{w.x, w.y}, {w.z, w.w}};
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const uint32_t A = pr[p][0], Bw = pr[p][1];
                const uint32_t ulo = (A & 0xFFFFu) | (Bw << 16);
                const uint32_t uhi = (A >> 16) | (Bw & 0xFFFF0000u);
                fkv_h2* dst = p == 0 ? v01 : v23;
                dst[0] = as_h2(((ulo << 6) & 0x03C003C0u) | 0x4C004C00u);
                dst[1] = as_h2(((ulo << 2) & 0x03C003C0u) | 0x4C004C00u);
                dst[2] = as_h2(((ulo >> 2) & 0x03C003C0u) | 0x4C004C00u);
                dst[3] = as_h2(((ulo >> 6) & 0x03C003C0u) | 0x4C004C00u);
                dst[4] = as_h2(((uhi << 6) & 0x03C003C0u) | 0x4C004C00u);
                dst[5] = as_h2(((uhi << 2) & 0x03C003C0u) | 0x4C004C00u);
                dst[6] = as_h2(((uhi >> 2) & 0x03C003C0u) | 0x4C004C00u);
                dst[7] = as_h2(((uhi >> 6) & 0x03C003C0u) | 0x4C004C00u);
            }
        } else {
            uint4 r[4];
            const int t0 = tile * kTile + j * GS + ph;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = t0 + NPH * i;
                if (kind == kNear) {
                    r[i] = ((const uint4*)((const uint16_t*)(a.blob + a.L.near_v) +
                                           (bkv * a.L.Na_pad + t) * D))[qb];
                } else {
                    r[i] = t < count ? ((const uint4*)(a.dec_v + (bkv * a.n_dec + t) * D))[qb]
                                     : make_uint4(0, 0, 0, 0);
                }
            }
            uint32_t ra[4] = {r[0].x, r[0].y, r[0].z, r[0].w};
            uint32_t rb[4] = {r[1].x, r[1].y, r[1].z, r[1].w};
            uint32_t rc[4] = {r[2].x, r[2].y, r[2].z, r[2].w};
            uint32_t rd[4] = {r[3].x, r[3].y, r[3].z, r[3].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                v01[2 * k] = as_h2((ra[k] & 0xFFFFu) | (rb[k] << 16));
                v01[2 * k + 1] = as_h2((ra[k] >> 16) | (rb[k] & 0xFFFF0000u));
                v23[2 * k] = as_h2((rc[k] & 0xFFFFu) | (rd[k] << 16));
                v23[2 * k + 1] = as_h2((rc[k] >> 16) | (rd[k] & 0xFFFF0000u));
            }
        }
#pragma unroll
        for (int g = 0; g < GG; g++) {
            uint2 pw;
            __builtin_memcpy(&pw, pl + g * kTile + j * GS + ph * 4, 8);
            const fkv_h2 p01 = as_h2(pw.x), p23 = as_h2(pw.y);
#pragma unroll
            for (int d = 0; d < 8; d++) {
                float acc = st.acc[g][d];
                acc = dot2(p01, v01[d], acc);
                acc = dot2(p23, v23[d], acc);
                st.acc[g][d] = acc;
            }
        }
    }
}

template <int D, int GG>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
    constexpr int NQ = D / 8, NPH = kWave / NQ, GS = 4 * NPH;
    constexpr int RS = Rec<D>::kSize;
    __shared__ __attribute__((aligned(16))) fkv_h2 qs[GG * (D / 2)];
    __shared__ __attribute__((aligned(16))) _Float16 pbuf[kWavesPerGroup][GG * kTile];
    __shared__ float wrec[kWavesPerGroup][GG * RS];

    const int split = blockIdx.x;
    const int kvh = blockIdx.y / a.head_groups;
    const int hgrp = blockIdx.y % a.head_groups;
    const int b = blockIdx.z;
    const int64_t bkv = (int64_t)b * a.L.Hkv + kvh;
    const int head0 = kvh * a.G + hgrp * GG;  // first q head of this workgroup
    const int ng = min(GG, a.G - hgrp * GG);   // heads actually served
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;

    // query heads -> LDS (fp16 pairs); heads beyond ng are zero
    for (int i = threadIdx.x; i < GG * (D / 2); i += blockDim.x) {
        const int g = i / (D / 2), e = i % (D / 2);
        uint32_t v = 0;
        if (g < ng) v = ((const uint32_t*)(a.q + ((int64_t)b * a.Hq + head0 + g) * D))[e];
        qs[i] = as_h2(v);
    }

    // split range over the virtual tile sequence, weighted by bytes per token
    const int nv = (int)((const uint32_t*)(a.blob + a.L.near_valid))[kvh];
    const int nt_near = (int)cdiv(nv, kTile);
    const int nt_far = (int)cdiv(a.L.F, kTile);
    const int nt_dec = (int)cdiv(a.n_dec, kTile);
    const int64_t wn = 4 * D, wf = (3 * D) / 2 + 4;  // bytes per near / far token
    const int64_t W = nt_near * wn + nt_far * wf + nt_dec * wn;
    auto first_tile_at = [&](int64_t x) -> int {
        if (x <= nt_near * wn) return (int)cdiv(x, wn);
        x -= nt_near * wn;
        if (x <= nt_far * wf) return nt_near + (int)cdiv(x, wf);
        x -= nt_far * wf;
        return nt_near + nt_far + (int)cdiv(x, wn);
    };
    const int k0 = first_tile_at(W * split / a.num_splits);
    const int k1 = first_tile_at(W * (split + 1) / a.num_splits);
    __syncthreads();

    WaveState<D, GG> st;
#pragma unroll
    for (int g = 0; g < GG; g++) {
        st.m[g] = -INFINITY;
        st.lsum[g] = 0.f;
        st.zsum[g] = 0.f;
        st.wsum[g] = 0.f;
        st.mn[g] = INFINITY;
        st.mx[g] = -INFINITY;
        st.arg[g] = INT_MAX;
#pragma unroll
        for (int d = 0; d < 8; d++) st.acc[g][d] = 0.f;
    }
    _Float16* pl = pbuf[wave];

    for (int k = k0 + wave; k < k1; k += kWavesPerGroup) {
        int kind, tile, count;
        if (k < nt_near) {
            kind = kNear; tile = k; count = nv;
        } else if (k < nt_near + nt_far) {
            kind = kFar; tile = k - nt_near; count = a.L.F;
        } else {
            kind = kDec; tile = k - nt_near - nt_far; count = a.n_dec;
        }
        // far V for this tile is loaded up front so its latency hides behind QK
        uint4 vfar[kTile / GS];
        if (kind == kFar) {
            const uint4* vb = (const uint4*)(a.blob + a.L.far_v) + (bkv * a.L.F_pad + (int64_t)tile * kTile) * D / 32;
#pragma unroll
            for (int j = 0; j < kTile / GS; j++) vfar[j] = vb[j * kWave + lane];
        }
        float s[GG];
        uint32_t sz;
        score_tile<D, GG>(a, kind, tile, bkv, count, qs, s, sz);

        const int tok = tile * kTile + lane;
        // spike bookkeeping (the V gate below does not affect it)
#pragma unroll
        for (int g = 0; g < GG; g++) {
            if (kind == kFar) {
                if (s[g] > st.mx[g]) { st.mx[g] = s[g]; st.arg[g] = tok; }
            } else {
                st.mn[g] = fminf(st.mn[g], s[g] == -INFINITY ? INFINITY : s[g]);
            }
        }
        // online softmax: one rescale per tile
        float p[GG];
        bool any = false;
#pragma unroll
        for (int g = 0; g < GG; g++) {
            const float tmax = wave_max(s[g]);
            const float m_new = fmaxf(st.m[g], tmax);
            if (m_new > st.m[g]) {
                const float alpha = __expf(st.m[g] - m_new);
                st.lsum[g] *= alpha;
                st.zsum[g] *= alpha;
                st.wsum[g] *= alpha;
#pragma unroll
                for (int d = 0; d < 8; d++) st.acc[g][d] *= alpha;
                st.m[g] = m_new;
            }
            float pg = 0.f;
            if (kind == kFar) {
                if (s[g] >= st.m[g] - 16.0f) pg = __expf(s[g] - st.m[g]);
            } else if (s[g] != -INFINITY) {
                pg = __expf(s[g] - st.m[g]);
            }
            p[g] = pg;
            any |= pg > 0.f;
        }
        const float vs = h2f((uint16_t)(sz & 0xFFFF));
        const float vz = h2f((uint16_t)(sz >> 16));
        const int rr = lane % GS;
        const int slot = (lane / GS) * GS + (rr % NPH) * 4 + rr / NPH;
#pragma unroll
        for (int g = 0; g < GG; g++) {
            st.lsum[g] += p[g];
            float w = p[g];
            if (kind == kFar) w = p[g] * vs;
            const _Float16 wh = (_Float16)w;
            if (kind == kFar) {
                // v = vs*(c - 7.5) + (vz + 7.5*vs); the accumulator receives
                // wh*(16 + c), so subtract 23.5*wh exactly via wsum
                st.zsum[g] += p[g] * (vz + 7.5f * vs);
                st.wsum[g] += (float)wh;
            }
            __builtin_memcpy(pl + g * kTile + slot, &wh, 2);
        }
        // whole tile gated away -> skip its V (wave-uniform)
        if (__builtin_amdgcn_ballot_w64(any) == 0) continue;
        // LDS ops of one wave complete in order: the weights just written are
        // visible to the reads below without a workgroup barrier
        __builtin_amdgcn_wave_barrier();
        pv_tile<D, GG>(a, kind, tile, bkv, count, pl, vfar, st);
        __builtin_amdgcn_wave_barrier();
    }

    // ---- wave reduction ----
    float* wr = wrec[wave];
#pragma unroll
    for (int g = 0; g < GG; g++) {
        float l = wave_sum(st.lsum[g]);
        float z = wave_sum(st.zsum[g]) - 23.5f * wave_sum(st.wsum[g]);
        float mn = wave_min(st.mn[g]);
        float mx = st.mx[g];
        int arg = st.arg[g];
        wave_argmax(mx, arg);
#pragma unroll
        for (int d = 0; d < 8; d++) {
            float v = st.acc[g][d];
#pragma unroll
            for (int o = NQ; o < kWave; o <<= 1) v += wave_xor(v, o);
            st.acc[g][d] = v + z;  // fold the INT4 zero-point term
        }
        if (lane == 0) {
            wr[g * RS + 0] = st.m[g];
            wr[g * RS + 1] = l;
            wr[g * RS + 2] = mn;
            wr[g * RS + 3] = mx;
            wr[g * RS + 4] = __int_as_float(arg);
        }
        if (lane < NQ) {
#pragma unroll
            for (int d = 0; d < 8; d++) wr[g * RS + Rec<D>::kHdr + lane * 8 + d] = st.acc[g][d];
        }
    }
    __syncthreads();

    // ---- merge the 4 waves (wave 0) into wrec[0] ----
    if (wave == 0) {
        for (int g = 0; g < GG; g++) {
            float M = -INFINITY;
            for (int w = 0; w < kWavesPerGroup; w++) M = fmaxf(M, wrec[w][g * RS]);
            float L = 0.f, mn = INFINITY, mx = -INFINITY;
            int arg = INT_MAX;
            float sc[kWavesPerGroup];
            for (int w = 0; w < kWavesPerGroup; w++) {
                const float mw = wrec[w][g * RS];
                sc[w] = mw == -INFINITY ? 0.f : __expf(mw - M);
                L += sc[w] * wrec[w][g * RS + 1];
                mn = fminf(mn, wrec[w][g * RS + 2]);
                const float fx = wrec[w][g * RS + 3];
                const int fa = __float_as_int(wrec[w][g * RS + 4]);
                if (fx > mx || (fx == mx && fa < arg)) { mx = fx; arg = fa; }
            }
            for (int d = lane; d < D; d += kWave) {
                float v = 0.f;
                for (int w = 0; w < kWavesPerGroup; w++) v += sc[w] * wrec[w][g * RS + Rec<D>::kHdr + d];
                wrec[0][g * RS + Rec<D>::kHdr + d] = v;
            }
            if (lane == 0) {
                wrec[0][g * RS + 0] = M;
                wrec[0][g * RS + 1] = L;
                wrec[0][g * RS + 2] = mn;
                wrec[0][g * RS + 3] = mx;
                wrec[0][g * RS + 4] = __int_as_float(arg);
            }
        }
    }
    __syncthreads();

    if (a.num_splits > 1) {
        // split partial -> workspace; merge_kernel combines the splits
        const int row = (int)(bkv * a.head_groups + hgrp);  // (b, kv_head, head group)
        float* dst = a.ws + ((int64_t)row * a.num_splits + split) * GG * RS;
        for (int i = threadIdx.x; i < GG * RS; i += blockDim.x) dst[i] = wrec[0][i];
        return;
    }
    finalize_rows<D>(a, wrec[0], GG, b, head0, ng);
}

// out = acc / l (fp16), spike flag and token for the ng heads of one record set
template <int D>
__device__ inline void finalize_rows(const AttnArgs& a, const float* fin, int GG_, int b, int head0, int ng) {
    constexpr int RS = Rec<D>::kSize;
    for (int i = threadIdx.x; i < ng * D; i += blockDim.x) {
        const int g = i / D, d = i % D;
        const float L = fin[g * RS + 1];
        const float inv_l = L > 0.f ? 1.0f / L : 0.f;
        a.out[((int64_t)b * a.Hq + head0 + g) * D + d] = f2h(fin[g * RS + Rec<D>::kHdr + d] * inv_l);
    }
    if ((int)threadIdx.x < ng) {
        const int g = threadIdx.x;
        const float mn = fin[g * RS + 2], mx = fin[g * RS + 3];
        const int arg = __float_as_int(fin[g * RS + 4]);
        const int64_t o = (int64_t)b * a.Hq + head0 + g;
        a.flags[o] = mx > mn + a.spike_margin ? 1 : 0;
        a.tokens[o] = mx == -INFINITY ? -1 : arg;
    }
    (void)GG_;
}

// Split-K merge (csrc/kernels/foveated_attn.metal:394-431 restated for
// partials in memory): one workgroup per (b, kv_head, head group).  The
// per-split maxima are rescaled to the global max; spike fields take the
// min / first-index max.
template <int D, int GG>
__global__ __launch_bounds__(256) void merge_kernel(AttnArgs a) {
    constexpr int RS = Rec<D>::kSize;
    constexpr int H = Rec<D>::kHdr;
    __shared__ float mrg[GG * RS];
    __shared__ float hdr[256][GG][H];  // per split: m, l, min_near, max_far, arg
    __shared__ float scl[GG][256];
    const int row = blockIdx.x;
    const int hgrp = row % a.head_groups;
    const int64_t bkv = row / a.head_groups;
    const int b = (int)(bkv / a.L.Hkv), kvh = (int)(bkv % a.L.Hkv);
    const int head0 = kvh * a.G + hgrp * GG;
    const int ng = min(GG, a.G - hgrp * GG);
    const float* src = a.ws + (int64_t)row * a.num_splits * GG * RS;
    const int ns = a.num_splits;  // <= 256
    // 1) every (split, head) header in one parallel round trip
    for (int i = threadIdx.x; i < ns * GG * H; i += blockDim.x) {
        const int sp = i / (GG * H), r = i % (GG * H), g = r / H, f = r % H;
        hdr[sp][g][f] = src[(int64_t)sp * GG * RS + g * RS + f];
    }
    __syncthreads();
    // 2) per-head global max, scales, normaliser and spike fields
    if (threadIdx.x < GG) {
        const int g = threadIdx.x;
        float M = -INFINITY;
        for (int sp = 0; sp < ns; sp++) M = fmaxf(M, hdr[sp][g][0]);
        float L = 0.f, mn = INFINITY, mx = -INFINITY;
        int arg = INT_MAX;
        for (int sp = 0; sp < ns; sp++) {
            const float mw = hdr[sp][g][0];
            const float f = mw == -INFINITY ? 0.f : __expf(mw - M);
            scl[g][sp] = f;
            L += f * hdr[sp][g][1];
            mn = fminf(mn, hdr[sp][g][2]);
            const float fx = hdr[sp][g][3];
            const int fa = __float_as_int(hdr[sp][g][4]);
            if (fx > mx || (fx == mx && fa < arg)) { mx = fx; arg = fa; }
        }
        mrg[g * RS + 0] = M;
        mrg[g * RS + 1] = L;
        mrg[g * RS + 2] = mn;
        mrg[g * RS + 3] = mx;
        mrg[g * RS + 4] = __int_as_float(arg);
    }
    __syncthreads();
    // 3) rescaled sum of the accumulators (independent loads per element)
    for (int i = threadIdx.x; i < GG * D; i += blockDim.x) {
        const int g = i / D, d = i % D;
        const float* col = src + g * RS + H + d;
        float v = 0.f;
#pragma unroll 8
        for (int sp = 0; sp < ns; sp++) v += scl[g][sp] * col[(int64_t)sp * GG * RS];
        mrg[g * RS + H + d] = v;
    }
    __syncthreads();
    finalize_rows<D>(a, mrg, GG, b, head0, ng);
}

}  // namespace fkv

// ---------------------------------------------------------------------------
// Host side: handle + launch
// ---------------------------------------------------------------------------

struct fkv_attn_impl {
    fkv::BlobLayout L;
    uint8_t* blob = nullptr;
    float margin = 0.f;
    float* ws = nullptr;          // split partials
    size_t ws_floats = 0;
    uint16_t* qbuf = nullptr;     // fp16 copy of non-fp16 queries
    size_t qbuf_n = 0;
    int device = 0;
};

namespace fkv {

constexpr int kMaxG = 8;  // query heads served per workgroup

typedef void (*AttnKernel)(AttnArgs);

template <int D>
static AttnKernel pick_kernel(int gg) {
    switch (gg) {
        case 1: return attn_kernel<D, 1>;
        case 2: return attn_kernel<D, 2>;
        case 3: return attn_kernel<D, 3>;
        case 4: return attn_kernel<D, 4>;
        case 5: return attn_kernel<D, 5>;
        case 6: return attn_kernel<D, 6>;
        case 7: return attn_kernel<D, 7>;
        default: return attn_kernel<D, 8>;
    }
}

template <int D>
static AttnKernel pick_merge(int gg) {
    switch (gg) {
        case 1: return merge_kernel<D, 1>;
        case 2: return merge_kernel<D, 2>;
        case 3: return merge_kernel<D, 3>;
        case 4: return merge_kernel<D, 4>;
        case 5: return merge_kernel<D, 5>;
        case 6: return merge_kernel<D, 6>;
        case 7: return merge_kernel<D, 7>;
        default: return merge_kernel<D, 8>;
    }
}

static int grid_for(int64_t n, int block) {
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
int plan_splits(const BlobLayout& L, int rows, int n_dec) {
    const int tiles = (int)(cdiv(L.Na, kTile) + cdiv(L.F, kTile) + cdiv(n_dec, kTile));
    const int target = env_int("FKV_TARGET_WGS", 1024);
    int s = (int)cdiv(target, rows > 0 ? rows : 1);
    const int cap = tiles / (2 * kWavesPerGroup);
    if (s > cap) s = cap;
    if (s > 256) s = 256;
    return s < 1 ? 1 : s;
}

}  // namespace fkv

using fkv::check_hip;
using fkv::set_error;

extern "C" {

struct fkv_attn : fkv_attn_impl {};

int fkv_attn_create(fkv_attn** out, int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F,
                    const void* near_k, const void* near_v, int32_t near_dtype,
                    const uint8_t* far_k, const uint8_t* far_v, const void* far_v_scale,
                    const void* far_v_zero, int32_t sz_dtype, const int32_t* near_valid,
                    float spike_margin, void* stream) {
    if (!out) return set_error("fkv_attn_create: out is NULL");
    *out = nullptr;
    if (B <= 0 || Hkv <= 0 || Na < 0 || F < 0)
        return set_error("fkv_attn_create: bad shape B=" + std::to_string(B) + " Hkv=" +
                         std::to_string(Hkv) + " Na=" + std::to_string(Na) + " F=" + std::to_string(F));
    if (D != 64 && D != 128) return set_error("fkv_attn_create: head dim must be 64 or 128, got " + std::to_string(D));
    if (near_dtype < FKV_F16 || near_dtype > FKV_F32 || sz_dtype < FKV_F16 || sz_dtype > FKV_F32)
        return set_error("fkv_attn_create: unsupported dtype");
    if ((Na > 0 && (!near_k || !near_v)) || (F > 0 && (!far_k || !far_v || !far_v_scale || !far_v_zero)) ||
        !near_valid)
        return set_error("fkv_attn_create: NULL tier array");
    hipStream_t st = (hipStream_t)stream;
    fkv_attn* h = new fkv_attn();
    h->L = fkv::make_layout(B, Hkv, D, Na, F);
    h->margin = spike_margin;
    int rc = check_hip(hipGetDevice(&h->device), "hipGetDevice");
    unsigned* bad = nullptr;
    if (!rc) rc = check_hip(hipMalloc(&h->blob, h->L.total), "hipMalloc(blob)");
    if (!rc) rc = check_hip(hipMalloc(&bad, sizeof(unsigned)), "hipMalloc(flag)");
    if (!rc) rc = check_hip(hipMemsetAsync(bad, 0, sizeof(unsigned), st), "hipMemsetAsync");
    if (!rc) rc = check_hip(hipMemsetAsync(h->blob, 0, h->L.total, st), "hipMemsetAsync(blob)");
    if (!rc) {
        const int blk = 256;
        const fkv::BlobLayout L = h->L;
        if (Na > 0)
            hipLaunchKernelGGL(fkv::pack_near_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * L.Na_pad * (D / 8), blk)),
                               dim3(blk), 0, st, near_k, near_v, near_dtype, L, h->blob);
        if (F > 0) {
            hipLaunchKernelGGL(fkv::pack_far_k_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * L.F_pad * (D / 16), blk)),
                               dim3(blk), 0, st, far_k, L, h->blob, bad);
            hipLaunchKernelGGL(fkv::pack_far_v_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * L.F_pad * (D / 8), blk)),
                               dim3(blk), 0, st, far_v, far_v_scale, far_v_zero, sz_dtype, L, h->blob);
        }
        hipLaunchKernelGGL(fkv::pack_valid_kernel, dim3(1), dim3(blk), 0, st, near_valid, Hkv, L, h->blob);
        rc = check_hip(hipGetLastError(), "pack kernels");
    }
    unsigned bad_h = 0;
    if (!rc) rc = check_hip(hipMemcpyAsync(&bad_h, bad, sizeof(unsigned), hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    if (!rc) rc = check_hip(hipStreamSynchronize(st), "hipStreamSynchronize");
    if (bad) (void)hipFree(bad);
    if (!rc && bad_h) {
        set_error("fkv_attn_create: far_k holds E4M3 NaN codes 0x7F/0xFF, which the reference encoder never emits");
        rc = FKV_EDATA;
    }
    if (rc) {
        fkv_attn_destroy(h);
        return rc;
    }
    *out = h;
    return FKV_OK;
}

int fkv_attn_call(fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq,
                  const void* decode_k, const void* decode_v, int32_t n_decode, void* out,
                  int32_t* spike_flags, int32_t* spike_tokens, void* stream) {
    if (!h || !query || !out || !spike_flags || !spike_tokens) return set_error("fkv_attn_call: NULL argument");
    const fkv::BlobLayout& L = h->L;
    if (Hq <= 0 || Hq % L.Hkv != 0)
        return set_error("fkv_attn_call: Hq=" + std::to_string(Hq) + " is not a multiple of H_kv=" + std::to_string(L.Hkv));
    if (n_decode < 0 || (n_decode > 0 && (!decode_k || !decode_v)))
        return set_error("fkv_attn_call: bad decode buffer");
    if (q_dtype < FKV_F16 || q_dtype > FKV_F32) return set_error("fkv_attn_call: unsupported query dtype");
    hipStream_t st = (hipStream_t)stream;
    const int G = Hq / L.Hkv;
    const int gg = G < fkv::kMaxG ? G : fkv::kMaxG;
    const int head_groups = (int)fkv::cdiv(G, gg);
    const int rows = L.B * L.Hkv * head_groups;
    const int splits = fkv::plan_splits(L, rows, n_decode);
    const uint16_t* q16 = (const uint16_t*)query;
    const int64_t qn = (int64_t)L.B * Hq * L.D;
    if (q_dtype != FKV_F16) {
        if ((size_t)qn > h->qbuf_n) {
            if (h->qbuf) (void)hipFree(h->qbuf);
            h->qbuf = nullptr;
            h->qbuf_n = 0;
            if (int rc = check_hip(hipMalloc(&h->qbuf, qn * 2), "hipMalloc(qbuf)")) return rc;
            h->qbuf_n = qn;
        }
        hipLaunchKernelGGL(fkv::cast_to_f16_kernel, dim3(fkv::grid_for(qn, 256)), dim3(256), 0, st, query,
                           q_dtype, qn, h->qbuf);
        q16 = h->qbuf;
    }
    const int RS = fkv::Rec<128>::kHdr + L.D;
    if (splits > 1) {
        const size_t need = (size_t)rows * splits * gg * RS;
        if (need > h->ws_floats) {
            if (h->ws) (void)hipFree(h->ws);
            h->ws = nullptr;
            h->ws_floats = 0;
            if (int rc = check_hip(hipMalloc(&h->ws, need * sizeof(float)), "hipMalloc(ws)")) return rc;
            h->ws_floats = need;
        }
    }
    fkv::AttnArgs a;
    a.blob = h->blob;
    a.L = L;
    a.q = q16;
    a.dec_k = (const uint16_t*)decode_k;
    a.dec_v = (const uint16_t*)decode_v;
    a.n_dec = n_decode;
    a.Hq = Hq;
    a.G = G;
    a.head_groups = head_groups;
    a.num_splits = splits;
    a.spike_margin = h->margin;
    a.inv_sqrt_d = (float)(1.0 / sqrt((double)L.D));
    a.out = (uint16_t*)out;
    a.flags = spike_flags;
    a.tokens = spike_tokens;
    a.ws = h->ws;
    fkv::AttnKernel k = L.D == 128 ? fkv::pick_kernel<128>(gg) : fkv::pick_kernel<64>(gg);
    hipLaunchKernelGGL(k, dim3(splits, L.Hkv * head_groups, L.B), dim3(fkv::kWave * fkv::kWavesPerGroup), 0, st, a);
    if (splits > 1) {
        fkv::AttnKernel m = L.D == 128 ? fkv::pick_merge<128>(gg) : fkv::pick_merge<64>(gg);
        hipLaunchKernelGGL(m, dim3(rows), dim3(256), 0, st, a);
    }
    return check_hip(hipGetLastError(), "attn_kernel launch");
}

int fkv_e4m3_decode(const uint8_t* codes, void* out_f16, int64_t n, void* stream) {
    if (n < 0 || n % 4 != 0 || (n > 0 && (!codes || !out_f16)))
        return set_error("fkv_e4m3_decode: n must be a multiple of 4 with non-NULL buffers");
    if (n == 0) return FKV_OK;
    hipLaunchKernelGGL(fkv::e4m3_decode_kernel, dim3(fkv::grid_for(n / 4, 256)), dim3(256), 0,
                       (hipStream_t)stream, codes, (uint16_t*)out_f16, n / 4);
    return check_hip(hipGetLastError(), "e4m3_decode_kernel launch");
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

void fkv_attn_destroy(fkv_attn* h) {
    if (!h) return;
    if (h->blob) (void)hipFree(h->blob);
    if (h->ws) (void)hipFree(h->ws);
    if (h->qbuf) (void)hipFree(h->qbuf);
    delete h;
}

}  // extern "C"
