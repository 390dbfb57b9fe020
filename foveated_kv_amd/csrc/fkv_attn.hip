// Fused two-tier split-K decode attention for gfx950 (fp8-E4M3 K / INT4 V far
// tier, fp16 near tier, fp16 decode buffer) and the per-layer device blob.
//
// Replaces the reference's FoveatedHandle + foveated_2tier Metal kernel
// (csrc/foveated_attn.cpp:83-254, csrc/kernels/foveated_attn.metal:181-432).
//
// Work decomposition: one workgroup of 4 waves per (batch, kv_head, split)
// serves up to 16 query heads of the GQA group, so each compressed byte is
// read from HBM once.  Both contractions of one kv head run on the matrix
// cores with v_mfma_f32_16x16x16_f16 (fp16 operands, fp32 accumulation):
//   scores  S[t][h] = K[t][:] . q[h][:]      A = K (16 tokens x 16 dims),
//                                             B = q (16 dims x 16 heads)
//   output  O[d][h] += V[t][d]^T . P[t][h]    A = V^T (16 dims x 16 tokens),
//                                             B = P (16 tokens x 16 heads)
// The score tile comes out of the first MFMA in exactly the register layout
// the second one takes as B, so softmax weights never leave registers.
// E4M3 keys are widened to fp16 with the native converter (exact); INT4
// values are widened exactly by inserting the nibble into an fp16 mantissa
// (16 + c), weights are p*scale, and the zero point and constant offsets
// are folded into per-head scalars.  The fp16 query is used unscaled (exact
// products); 1/sqrt(D) is applied to the fp32 scores.
// The blob stores every tier pre-arranged in these operand layouts so each
// lane's operand bytes are contiguous and every wave load is a contiguous
// 1 KB.  Split partials are merged by a small second kernel.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstring>

#include "fkv_attn.h"
#include "fkv_common.h"

typedef _Float16 fkv_h4 __attribute__((ext_vector_type(4)));
typedef float fkv_f4 __attribute__((ext_vector_type(4)));

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

// One thread per (bkv, 16-token group, lane).  Near K lane (kg, m) holds
// token m of the group, dims 16s + 4kg + i (s = 0..D/16-1, i = 0..3); near V
// lane (kg, m) holds dim 16j + m of tokens 4kg + i.  Slots >= Na are zero.
__global__ void pack_near_kernel(const void* __restrict__ nk, const void* __restrict__ nv,
                                 int dtype, BlobLayout L, uint8_t* __restrict__ blob) {
    const int D = L.D, NB = D / 16;
    const int64_t groups = L.Na_pad / 16;
    const int64_t n = (int64_t)L.B * L.Hkv * groups * kWave;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % kWave);
        const int64_t r = i / kWave;
        const int grp = (int)(r % groups);
        const int64_t bkv = r / groups;
        const int m = lane & 15, kg = lane >> 4;
        uint16_t* kd = (uint16_t*)(blob + L.near_k) + bkv * (int64_t)L.Na_pad * D +
                       (int64_t)grp * 16 * D + lane * (D / 4);
        uint16_t* vd = (uint16_t*)(blob + L.near_v) + bkv * (int64_t)L.Na_pad * D +
                       (int64_t)grp * 16 * D + lane * (D / 4);
        const int tk = grp * 16 + m;
        for (int s = 0; s < NB; s++)
            for (int e = 0; e < 4; e++)
                kd[s * 4 + e] = tk < L.Na ? load_as_f16(nk, (bkv * L.Na + tk) * D + 16 * s + 4 * kg + e, dtype) : 0;
        for (int j = 0; j < NB; j++)
            for (int e = 0; e < 4; e++) {
                const int tv = grp * 16 + 4 * kg + e;
                vd[j * 4 + e] = tv < L.Na ? load_as_f16(nv, (bkv * L.Na + tv) * D + 16 * j + m, dtype) : 0;
            }
    }
}

// Far K codes in the same operand layout as near K (bytes); exponent-0
// codes are written as signed zero (the reference LUT ignores their
// mantissa); NaN codes 0x7F/0xFF are reported through *bad.
__global__ void pack_far_k_kernel(const uint8_t* __restrict__ fk, BlobLayout L,
                                  uint8_t* __restrict__ blob, unsigned* __restrict__ bad) {
    const int D = L.D, NB = D / 16;
    const int64_t groups = L.F_pad / 16;
    const int64_t n = (int64_t)L.B * L.Hkv * groups * kWave;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % kWave);
        const int64_t r = i / kWave;
        const int grp = (int)(r % groups);
        const int64_t bkv = r / groups;
        const int m = lane & 15, kg = lane >> 4;
        const int t = grp * 16 + m;
        uint8_t* dst = blob + L.far_k + bkv * (int64_t)L.F_pad * D + (int64_t)grp * 16 * D + lane * (D / 4);
        for (int s = 0; s < NB; s++)
            for (int e = 0; e < 4; e++) {
                uint8_t b = 0;
                if (t < L.F) {
                    b = fk[(bkv * L.F + t) * D + 16 * s + 4 * kg + e];
                    if ((b & 0x7F) == 0x7F) atomicOr(bad, 1u);
                    if ((b & 0x78) == 0) b &= 0x80;
                }
                dst[s * 4 + e] = b;
            }
    }
}

// Far V nibbles: lane (kg, m) of a 16-token group holds D/32 dwords; dword u
// covers blocks 2u (bits 0-7, 16-23) and 2u+1 (bits 8-15, 24-31) at dim
// 16*block + m, with token 4kg+e at bit 16*(e&1) + 4*(e>>1) of its byte pair.
// Scale/zero -> one u32 per token.
__global__ void pack_far_v_kernel(const uint8_t* __restrict__ fv, const void* __restrict__ fvs,
                                  const void* __restrict__ fvz, int sz_dtype, BlobLayout L,
                                  uint8_t* __restrict__ blob) {
    const int D = L.D, NW = D / 32;
    const int64_t groups = L.F_pad / 16;
    const int64_t n = (int64_t)L.B * L.Hkv * groups * kWave;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % kWave);
        const int64_t r = i / kWave;
        const int grp = (int)(r % groups);
        const int64_t bkv = r / groups;
        const int m = lane & 15, kg = lane >> 4;
        uint32_t* dst = (uint32_t*)(blob + L.far_v + bkv * (int64_t)L.F_pad * D / 2) +
                        (int64_t)grp * 2 * D + lane * NW;
        for (int u = 0; u < NW; u++) {
            uint32_t w = 0;
            for (int bp = 0; bp < 2; bp++)
                for (int e = 0; e < 4; e++) {
                    const int t = grp * 16 + 4 * kg + e;
                    const int d = (2 * u + bp) * 16 + m;
                    uint32_t c = 0;
                    if (t < L.F) c = (fv[(bkv * L.F + t) * (D / 2) + d / 2] >> (4 * (d & 1))) & 15u;
                    w |= c << (bp * 8 + (e & 1) * 16 + (e >> 1) * 4);
                }
            dst[u] = w;
        }
        if (kg == 0) {
            const int t = grp * 16 + m;
            uint32_t sz = 0;
            if (t < L.F) {
                const int64_t k = bkv * L.F + t;
                sz = (uint32_t)load_as_f16(fvs, k, sz_dtype) | ((uint32_t)load_as_f16(fvz, k, sz_dtype) << 16);
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

constexpr int kHeads = 16;  // query heads per workgroup row (MFMA N)
constexpr int kHdr = 5;     // record header: m, l, min_near, max_far, first argmax
constexpr int kMaxSplits = 64;

struct AttnArgs {
    const uint8_t* blob;
    BlobLayout L;
    const uint16_t* q;      // (B, Hq, D) fp16
    const uint16_t* dec_k;  // (B, Hkv, n_dec, D) fp16 rows
    const uint16_t* dec_v;
    int n_dec;
    int Hq;
    int G;            // query heads per kv head
    int head_groups;  // workgroup rows per kv head (ceil(G / 16))
    int num_splits;
    float spike_margin;
    float inv_sqrt_d;
    uint16_t* out;  // (B, Hq, D) fp16
    int32_t* flags;
    int32_t* tokens;
    float* ws;  // split partials: [row][split][ng][kHdr + D]
};

__device__ inline fkv_f4 mfma16(fkv_h4 a, fkv_h4 b, fkv_f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ inline fkv_h4 h4_of(uint32_t lo, uint32_t hi) {
    uint2 u = make_uint2(lo, hi);
    return __builtin_bit_cast(fkv_h4, u);
}

// Four E4M3 codes -> fp16 A operand (dims 4kg + 0..3 of one k-step)
__device__ inline fkv_h4 e4m3x4(uint32_t w) {
    return h4_of(as_u32(e4m3x2_to_h2(w, false)), as_u32(e4m3x2_to_h2(w, true)));
}

// INT4 dword -> A operand of block 2u (bp = 0) or 2u+1 (bp = 1): (16 + c)
// for tokens 4kg + 0..3, exact.
__device__ inline fkv_h4 int4x4(uint32_t w, int bp) {
    const uint32_t a = bp ? ((w >> 2) & 0x03C003C0u) : ((w << 6) & 0x03C003C0u);
    const uint32_t b = bp ? ((w >> 6) & 0x03C003C0u) : ((w << 2) & 0x03C003C0u);
    return h4_of(a | 0x4C004C00u, b | 0x4C004C00u);
}

template <int D>
struct Lane {
    float m, lsum, zsum, wsum, mn, mx;
    int arg;
    fkv_f4 acc[D / 16];
};

template <int D>
__device__ inline void finalize_rows(const AttnArgs& a, const float* fin, int b, int head0, int ng);

// Online softmax + P.V for NG 16-token groups whose scores sc[g][e] (token
// 4kg+e of group g, head m) are computed.  vop(g, j) yields the A operand
// of block j of group g; far tiles pass their per-token scale/zero.
template <int D, int NG, bool FAR, typename VOp>
__device__ inline void softmax_pv(Lane<D>& st, const float (&sc)[NG][4], const uint32_t (&sz)[NG][4],
                                  VOp vop) {
    constexpr int NB = D / 16;
    float cmax = -INFINITY;
#pragma unroll
    for (int g = 0; g < NG; g++)
#pragma unroll
        for (int e = 0; e < 4; e++) cmax = fmaxf(cmax, sc[g][e]);
    cmax = fmaxf(cmax, wave_xor(cmax, 16));
    cmax = fmaxf(cmax, wave_xor(cmax, 32));
    const float m_new = fmaxf(st.m, cmax);
    if (__builtin_amdgcn_ballot_w64(m_new > st.m)) {
        const float alpha = m_new > st.m ? __expf(st.m - m_new) : 1.0f;
        st.lsum *= alpha;
        st.zsum *= alpha;
        st.wsum *= alpha;
#pragma unroll
        for (int j = 0; j < NB; j++) st.acc[j] *= alpha;
        st.m = m_new;
    }
    fkv_h4 bw[NG];
    bool any = false;
#pragma unroll
    for (int g = 0; g < NG; g++) {
        _Float16 wh[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float s = sc[g][e];
            float p = 0.f;
            if (FAR) {
                if (s >= st.m - 16.0f) p = __expf(s - st.m);  // score-gated V
            } else if (s != -INFINITY) {
                p = __expf(s - st.m);
            }
            st.lsum += p;
            if (FAR) {
                const float vs = h2f((uint16_t)(sz[g][e] & 0xFFFF));
                const float vz = h2f((uint16_t)(sz[g][e] >> 16));
                wh[e] = (_Float16)(p * vs);
                // value = vs*(c - 7.5) + (vz + 7.5*vs); the MFMA sees wh*(16 + c)
                st.zsum += p * (vz + 7.5f * vs);
                st.wsum += (float)wh[e];
            } else {
                wh[e] = (_Float16)p;
            }
            any |= p > 0.f;
        }
        bw[g] = fkv_h4{wh[0], wh[1], wh[2], wh[3]};
    }
    if (__builtin_amdgcn_ballot_w64(any) == 0) return;  // whole chunk gated away
#pragma unroll
    for (int g = 0; g < NG; g++)
#pragma unroll
        for (int j = 0; j < NB; j++) st.acc[j] = mfma16(vop(g, j), bw[g], st.acc[j]);
}

template <int D>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
    constexpr int NB = D / 16;  // 16-dim k-steps of QK == 16-dim blocks of P.V
    constexpr int RS = kHdr + D;
    __shared__ float wrec[kWavesPerGroup][kHeads * RS];

    const int split = blockIdx.x;
    const int kvh = blockIdx.y / a.head_groups;
    const int hgrp = blockIdx.y % a.head_groups;
    const int b = blockIdx.z;
    const int64_t bkv = (int64_t)b * a.L.Hkv + kvh;
    const int head0 = kvh * a.G + hgrp * kHeads;
    const int ng = min(kHeads, a.G - hgrp * kHeads);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int m = lane & 15, kg = lane >> 4;

    // query as the B operand of the score MFMA: head m, dims 16s + 4kg + 0..3
    fkv_h4 qb[NB];
#pragma unroll
    for (int s = 0; s < NB; s++) {
        uint2 v = make_uint2(0, 0);
        if (m < ng) v = *(const uint2*)(a.q + ((int64_t)b * a.Hq + head0 + m) * D + 16 * s + 4 * kg);
        qb[s] = __builtin_bit_cast(fkv_h4, v);
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

    Lane<D> st;
    st.m = -INFINITY;
    st.lsum = st.zsum = st.wsum = 0.f;
    st.mn = INFINITY;
    st.mx = -INFINITY;
    st.arg = INT_MAX;
#pragma unroll
    for (int j = 0; j < NB; j++) st.acc[j] = fkv_f4{0.f, 0.f, 0.f, 0.f};

    for (int k = k0 + wave; k < k1; k += kWavesPerGroup) {
        if (k >= nt_near && k < nt_near + nt_far) {
            // ---------------- far tile: 4 groups of 16 tokens ----------------
            const int tile = k - nt_near;
            const int64_t g0 = (int64_t)tile * 4;  // first group
            const uint8_t* kb = a.blob + a.L.far_k + bkv * (int64_t)a.L.F_pad * D + g0 * 16 * D + lane * (D / 4);
            const uint32_t* vb = (const uint32_t*)(a.blob + a.L.far_v + bkv * (int64_t)a.L.F_pad * D / 2) +
                                 g0 * 2 * D + lane * (D / 32);
            const uint32_t* zb = (const uint32_t*)(a.blob + a.L.far_sz) + bkv * a.L.F_pad + g0 * 16 + 4 * kg;
            uint32_t kw[4][NB], vw[4][NB / 2], sz[4][4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
#pragma unroll
                for (int q4 = 0; q4 < NB / 4; q4++) {
                    const uint4 x = *(const uint4*)(kb + g * 16 * D + q4 * 16);
                    kw[g][4 * q4] = x.x; kw[g][4 * q4 + 1] = x.y; kw[g][4 * q4 + 2] = x.z; kw[g][4 * q4 + 3] = x.w;
                }
                if constexpr (NB / 2 == 4) {
                    const uint4 x = *(const uint4*)(vb + g * 2 * D);
                    vw[g][0] = x.x; vw[g][1] = x.y; vw[g][2] = x.z; vw[g][3] = x.w;
                } else {
                    const uint2 x = *(const uint2*)(vb + g * 2 * D);
                    vw[g][0] = x.x; vw[g][1] = x.y;
                }
                const uint4 z = *(const uint4*)(zb + g * 16);
                sz[g][0] = z.x; sz[g][1] = z.y; sz[g][2] = z.z; sz[g][3] = z.w;
            }
            float sc[4][4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                fkv_f4 acc = fkv_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < NB; s++) acc = mfma16(e4m3x4(kw[g][s]), qb[s], acc);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = tile * kTile + g * 16 + 4 * kg + e;
                    const float s = acc[e] * a.inv_sqrt_d;
                    const bool ok = t < a.L.F;
                    sc[g][e] = ok ? s : -INFINITY;
                    if (ok && s > st.mx) { st.mx = s; st.arg = t; }  // first index of the max
                }
            }
            softmax_pv<D, 4, true>(st, sc, sz, [&](int g, int j) { return int4x4(vw[g][j >> 1], j & 1); });
        } else {
            // ---------- fp16 tile (near slots or decode rows): 2 x 2 groups ----------
            const bool near = k < nt_near;
            const int tile = near ? k : k - nt_near - nt_far;
            const int count = near ? nv : a.n_dec;
#pragma unroll 1
            for (int half = 0; half < 2; half++) {
                const int gbase = tile * 4 + half * 2;  // first 16-token group
                uint32_t kw[2][2 * NB], vw[2][2 * NB];
                if (near) {
                    const uint16_t* kb = (const uint16_t*)(a.blob + a.L.near_k) + bkv * (int64_t)a.L.Na_pad * D +
                                         (int64_t)gbase * 16 * D + lane * (D / 4);
                    const uint16_t* vb = (const uint16_t*)(a.blob + a.L.near_v) + bkv * (int64_t)a.L.Na_pad * D +
                                         (int64_t)gbase * 16 * D + lane * (D / 4);
#pragma unroll
                    for (int g = 0; g < 2; g++)
#pragma unroll
                        for (int q4 = 0; q4 < NB / 2; q4++) {
                            const uint4 x = *(const uint4*)(kb + g * 16 * D + q4 * 8);
                            const uint4 y = *(const uint4*)(vb + g * 16 * D + q4 * 8);
                            kw[g][4 * q4] = x.x; kw[g][4 * q4 + 1] = x.y; kw[g][4 * q4 + 2] = x.z; kw[g][4 * q4 + 3] = x.w;
                            vw[g][4 * q4] = y.x; vw[g][4 * q4 + 1] = y.y; vw[g][4 * q4 + 2] = y.z; vw[g][4 * q4 + 3] = y.w;
                        }
                } else {
                    // decode rows are row-major (B, Hkv, n_dec, D): gather operands
#pragma unroll
                    for (int g = 0; g < 2; g++) {
                        const int tk = (gbase + g) * 16 + m;
                        const uint16_t* kr = a.dec_k + (bkv * a.n_dec + (tk < count ? tk : 0)) * D;
#pragma unroll
                        for (int s = 0; s < NB; s++) {
                            const uint2 x = tk < count ? *(const uint2*)(kr + 16 * s + 4 * kg) : make_uint2(0, 0);
                            kw[g][2 * s] = x.x;
                            kw[g][2 * s + 1] = x.y;
                        }
#pragma unroll
                        for (int j = 0; j < NB; j++) {
                            uint16_t hv[4];
#pragma unroll
                            for (int e = 0; e < 4; e++) {
                                const int tv = (gbase + g) * 16 + 4 * kg + e;
                                hv[e] = tv < count ? a.dec_v[(bkv * a.n_dec + tv) * D + 16 * j + m] : (uint16_t)0;
                            }
                            vw[g][2 * j] = hv[0] | ((uint32_t)hv[1] << 16);
                            vw[g][2 * j + 1] = hv[2] | ((uint32_t)hv[3] << 16);
                        }
                    }
                }
                float sc[2][4];
                uint32_t szd[2][4] = {};
#pragma unroll
                for (int g = 0; g < 2; g++) {
                    fkv_f4 acc = fkv_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int s = 0; s < NB; s++) acc = mfma16(h4_of(kw[g][2 * s], kw[g][2 * s + 1]), qb[s], acc);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int t = (gbase + g) * 16 + 4 * kg + e;
                        const float s = acc[e] * a.inv_sqrt_d;
                        const bool ok = t < count;
                        sc[g][e] = ok ? s : -INFINITY;
                        if (ok) st.mn = fminf(st.mn, s);
                    }
                }
                softmax_pv<D, 2, false>(st, sc, szd,
                                        [&](int g, int j) { return h4_of(vw[g][2 * j], vw[g][2 * j + 1]); });
            }
        }
    }

    // ---- per-head reduction over the 4 lanes (kg) sharing head m ----
    float l = st.lsum, z = st.zsum, ws = st.wsum, mn = st.mn, mx = st.mx;
    int arg = st.arg;
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) {
        l += wave_xor(l, o);
        z += wave_xor(z, o);
        ws += wave_xor(ws, o);
        mn = fminf(mn, wave_xor(mn, o));
        const float ox = wave_xor(mx, o);
        const int oa = wave_xor(arg, o);
        if (ox > mx || (ox == mx && oa < arg)) { mx = ox; arg = oa; }
    }
    z -= 23.5f * ws;  // remove the +16 INT4 decode offset and the 7.5 centring
    float* wr = wrec[wave];
    if (m < ng) {
        if (kg == 0) {
            wr[m * RS + 0] = st.m;
            wr[m * RS + 1] = l;
            wr[m * RS + 2] = mn;
            wr[m * RS + 3] = mx;
            wr[m * RS + 4] = __int_as_float(arg);
        }
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) wr[m * RS + kHdr + 16 * j + 4 * kg + e] = st.acc[j][e] + z;
    }
    __syncthreads();

    // ---- merge the 4 waves into wrec[0] ----
    for (int h = wave; h < ng; h += kWavesPerGroup) {
        float M = -INFINITY;
        for (int w = 0; w < kWavesPerGroup; w++) M = fmaxf(M, wrec[w][h * RS]);
        float sc[kWavesPerGroup];
        float L = 0.f, mn2 = INFINITY, mx2 = -INFINITY;
        int arg2 = INT_MAX;
        for (int w = 0; w < kWavesPerGroup; w++) {
            const float mw = wrec[w][h * RS];
            sc[w] = mw == -INFINITY ? 0.f : __expf(mw - M);
            L += sc[w] * wrec[w][h * RS + 1];
            mn2 = fminf(mn2, wrec[w][h * RS + 2]);
            const float fx = wrec[w][h * RS + 3];
            const int fa = __float_as_int(wrec[w][h * RS + 4]);
            if (fx > mx2 || (fx == mx2 && fa < arg2)) { mx2 = fx; arg2 = fa; }
        }
        for (int d = lane; d < D; d += kWave) {
            float v = 0.f;
            for (int w = 0; w < kWavesPerGroup; w++) v += sc[w] * wrec[w][h * RS + kHdr + d];
            wrec[0][h * RS + kHdr + d] = v;
        }
        if (lane == 0) {
            wrec[0][h * RS + 0] = M;
            wrec[0][h * RS + 1] = L;
            wrec[0][h * RS + 2] = mn2;
            wrec[0][h * RS + 3] = mx2;
            wrec[0][h * RS + 4] = __int_as_float(arg2);
        }
    }
    __syncthreads();

    if (a.num_splits > 1) {
        const int row = (int)(bkv * a.head_groups + hgrp);  // (b, kv_head, head group)
        float* dst = a.ws + ((int64_t)row * a.num_splits + split) * ng * RS;
        for (int i = threadIdx.x; i < ng * RS; i += blockDim.x) dst[i] = wrec[0][i];
        return;
    }
    finalize_rows<D>(a, wrec[0], b, head0, ng);
}

// out = acc / l (fp16), spike flag and token for ng heads of one record set
template <int D>
__device__ inline void finalize_rows(const AttnArgs& a, const float* fin, int b, int head0, int ng) {
    constexpr int RS = kHdr + D;
    for (int i = threadIdx.x; i < ng * D; i += blockDim.x) {
        const int g = i / D, d = i % D;
        const float L = fin[g * RS + 1];
        const float inv_l = L > 0.f ? 1.0f / L : 0.f;
        a.out[((int64_t)b * a.Hq + head0 + g) * D + d] = f2h(fin[g * RS + kHdr + d] * inv_l);
    }
    if ((int)threadIdx.x < ng) {
        const int g = threadIdx.x;
        const float mn = fin[g * RS + 2], mx = fin[g * RS + 3];
        const int arg = __float_as_int(fin[g * RS + 4]);
        const int64_t o = (int64_t)b * a.Hq + head0 + g;
        a.flags[o] = mx > mn + a.spike_margin ? 1 : 0;
        a.tokens[o] = mx == -INFINITY ? -1 : arg;
    }
}

// Split-K merge (csrc/kernels/foveated_attn.metal:394-431 restated for
// partials in memory): one workgroup per (b, kv_head, head group).  Split
// maxima are rescaled to the global max; spike fields take the min and the
// first-index max.
template <int D>
__global__ __launch_bounds__(256) void merge_kernel(AttnArgs a) {
    constexpr int RS = kHdr + D;
    __shared__ float mrg[kHeads * RS];
    __shared__ float hdr[kMaxSplits][kHeads][kHdr];
    __shared__ float scl[kHeads][kMaxSplits];
    const int row = blockIdx.x;
    const int hgrp = row % a.head_groups;
    const int64_t bkv = row / a.head_groups;
    const int b = (int)(bkv / a.L.Hkv), kvh = (int)(bkv % a.L.Hkv);
    const int head0 = kvh * a.G + hgrp * kHeads;
    const int ng = min(kHeads, a.G - hgrp * kHeads);
    const int ns = a.num_splits;  // <= kMaxSplits
    const float* src = a.ws + (int64_t)row * ns * ng * RS;
    for (int i = threadIdx.x; i < ns * ng * kHdr; i += blockDim.x) {
        const int sp = i / (ng * kHdr), r = i % (ng * kHdr), g = r / kHdr, f = r % kHdr;
        hdr[sp][g][f] = src[(int64_t)sp * ng * RS + g * RS + f];
    }
    __syncthreads();
    if ((int)threadIdx.x < ng) {
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
    for (int i = threadIdx.x; i < ng * D; i += blockDim.x) {
        const int g = i / D, d = i % D;
        const float* col = src + g * RS + kHdr + d;
        float v = 0.f;
#pragma unroll 8
        for (int sp = 0; sp < ns; sp++) v += scl[g][sp] * col[(int64_t)sp * ng * RS];
        mrg[g * RS + kHdr + d] = v;
    }
    __syncthreads();
    finalize_rows<D>(a, mrg, b, head0, ng);
}

}  // namespace fkv

// ---------------------------------------------------------------------------
// Host side: handle + launch
// ---------------------------------------------------------------------------

struct fkv_attn_impl {
    fkv::BlobLayout L;
    uint8_t* blob = nullptr;
    float margin = 0.f;
    float* ws = nullptr;  // split partials
    size_t ws_floats = 0;
    uint16_t* qbuf = nullptr;  // fp16 copy of non-fp16 queries
    size_t qbuf_n = 0;
    int device = 0;
};

namespace fkv {

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
    if (s > kMaxSplits) s = kMaxSplits;
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
            hipLaunchKernelGGL(fkv::pack_near_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * (L.Na_pad / 16) * 64, blk)),
                               dim3(blk), 0, st, near_k, near_v, near_dtype, L, h->blob);
        if (F > 0) {
            hipLaunchKernelGGL(fkv::pack_far_k_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * (L.F_pad / 16) * 64, blk)),
                               dim3(blk), 0, st, far_k, L, h->blob, bad);
            hipLaunchKernelGGL(fkv::pack_far_v_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * (L.F_pad / 16) * 64, blk)),
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
    const int head_groups = (int)fkv::cdiv(G, fkv::kHeads);
    const int ng_max = G < fkv::kHeads ? G : fkv::kHeads;
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
    if (splits > 1) {
        const size_t need = (size_t)rows * splits * ng_max * (fkv::kHdr + L.D);
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
    const dim3 grid(splits, L.Hkv * head_groups, L.B), block(fkv::kWave * fkv::kWavesPerGroup);
    if (L.D == 128) hipLaunchKernelGGL(fkv::attn_kernel<128>, grid, block, 0, st, a);
    else hipLaunchKernelGGL(fkv::attn_kernel<64>, grid, block, 0, st, a);
    if (splits > 1) {
        if (L.D == 128) hipLaunchKernelGGL(fkv::merge_kernel<128>, dim3(rows), dim3(256), 0, st, a);
        else hipLaunchKernelGGL(fkv::merge_kernel<64>, dim3(rows), dim3(256), 0, st, a);
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
