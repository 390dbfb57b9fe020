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
        uint8_t* dst = blob + L.far_k + bkv * (int64_t)L.F_pad * D;
        for (int e = 0; e < 16; e++) {
            const int d = blk * 16 + e;
            uint8_t b = 0;
            if (t < L.F) {
                b = fk[(bkv * L.F + t) * D + d];
                if ((b & 0x7F) == 0x7F) atomicOr(bad, 1u);
                if ((b & 0x78) == 0) b &= 0x80;
            }
            dst[far_k_index(t, d, D)] = b;
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
        ((uint32_t*)(blob + L.far_v + bkv * (int64_t)L.F_pad * D / 2))[w] = word;
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
        ((uint32_t*)(blob + L.far_sz))[bkv * L.F_pad + t] = sz;
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

constexpr int kHeads = 16;  // query heads per workgroup row: up to 4 quads of 4
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

// v_mfma_f32_4x4x4f16: 16 independent 4x4x4 blocks; lane l supplies row /
// column l%4 of block l/4.  cbsz = 4, abid = s broadcasts block s's A.
template <int ABID>
__device__ inline fkv_f4 mfma4(fkv_h4 a, fkv_h4 b, fkv_f4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 4, ABID, 0);
}
__device__ inline fkv_f4 mfma4_local(fkv_h4 a, fkv_h4 b, fkv_f4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 0);
}

__device__ inline fkv_h4 h4_of(uint32_t lo, uint32_t hi) {
    uint2 u = make_uint2(lo, hi);
    return __builtin_bit_cast(fkv_h4, u);
}

// Four E4M3 codes -> fp16 (dims 4s..4s+3 of one token), exact.
__device__ inline fkv_h4 e4m3x4(uint32_t w) {
    return h4_of(as_u32(e4m3x2_to_h2(w, false)), as_u32(e4m3x2_to_h2(w, true)));
}

// INT4 dword -> the 4 tokens of 4-token group 2u (bp = 0) or 2u+1 (bp = 1)
// as fp16 (16 + c), exact: the nibble lands in mantissa bits 6..9 of an
// exponent-19 half.
__device__ inline fkv_h4 int4x4(uint32_t w, int bp) {
    const uint32_t a = bp ? ((w >> 2) & 0x03C003C0u) : ((w << 6) & 0x03C003C0u);
    const uint32_t b = bp ? ((w >> 6) & 0x03C003C0u) : ((w << 2) & 0x03C003C0u);
    return h4_of(a | 0x4C004C00u, b | 0x4C004C00u);
}

// broadcast lane i of each lane quad (DPP quad_perm)
template <int I>
__device__ inline float quad_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), I * 0x55, 0xF, 0xF, false));
}

template <int D, int NQ>
struct Lane {
    // per head quad: this lane tracks head 4*qd + (lane % 4)
    float m[NQ], lsum[NQ], zsum[NQ], wsum[NQ], mn[NQ], mx[NQ];
    int arg[NQ];
    fkv_f4 acc[NQ][D / 64];  // acc[qd][dh][i] = O[head 4qd+i][dim 64dh + lane]
};

enum TileKind { kNear = 0, kFar = 1, kDec = 2 };

template <int D>
__device__ inline void finalize_rows(const AttnArgs& a, const float* fin, int b, int head0, int ng);

// Online softmax of one 64-token tile for head quad qd (scores s[e] of
// tokens 4*(lane/4) + e, head 4qd + lane%4), then P.V: 16 broadcast MFMAs
// per 64-dim half, A = the weights of 4-token group g (abid = g), B = the
// values of that group at dim 64dh + lane.
template <int D, int NQ, bool FAR, typename VOp>
__device__ inline void softmax_pv(Lane<D, NQ>& st, int qd, const float (&s)[4], const uint32_t (&sz)[4],
                                  VOp vop) {
    constexpr int NH = D / 64;
    float cmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
#pragma unroll
    for (int o = 4; o <= 32; o <<= 1) cmax = fmaxf(cmax, wave_xor(cmax, o));
    const float m_new = fmaxf(st.m[qd], cmax);
    if (__builtin_amdgcn_ballot_w64(m_new > st.m[qd])) {
        const float alpha = m_new > st.m[qd] ? __expf(st.m[qd] - m_new) : 1.0f;
        st.lsum[qd] *= alpha;
        st.zsum[qd] *= alpha;
        st.wsum[qd] *= alpha;
        const float a0 = quad_bcast<0>(alpha), a1 = quad_bcast<1>(alpha);
        const float a2 = quad_bcast<2>(alpha), a3 = quad_bcast<3>(alpha);
#pragma unroll
        for (int dh = 0; dh < NH; dh++) {
            st.acc[qd][dh][0] *= a0;
            st.acc[qd][dh][1] *= a1;
            st.acc[qd][dh][2] *= a2;
            st.acc[qd][dh][3] *= a3;
        }
        st.m[qd] = m_new;
    }
    _Float16 wh[4];
    bool any = false;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float p = 0.f;
        if (FAR) {
            if (s[e] >= st.m[qd] - 16.0f) p = __expf(s[e] - st.m[qd]);  // score-gated V
        } else if (s[e] != -INFINITY) {
            p = __expf(s[e] - st.m[qd]);
        }
        st.lsum[qd] += p;
        if (FAR) {
            const float vs = h2f((uint16_t)(sz[e] & 0xFFFF));
            const float vz = h2f((uint16_t)(sz[e] >> 16));
            wh[e] = (_Float16)(p * vs);
            // value = vs*(c - 7.5) + (vz + 7.5*vs); the MFMA sees wh*(16 + c)
            st.zsum[qd] += p * (vz + 7.5f * vs);
            st.wsum[qd] += (float)wh[e];
        } else {
            wh[e] = (_Float16)p;
        }
        any |= p > 0.f;
    }
    if (__builtin_amdgcn_ballot_w64(any) == 0) return;  // whole tile gated away
    const fkv_h4 w4 = fkv_h4{wh[0], wh[1], wh[2], wh[3]};
#pragma unroll
    for (int dh = 0; dh < NH; dh++) {
        fkv_f4 acc = st.acc[qd][dh];
        acc = mfma4<0>(w4, vop(0, dh), acc);
        acc = mfma4<1>(w4, vop(1, dh), acc);
        acc = mfma4<2>(w4, vop(2, dh), acc);
        acc = mfma4<3>(w4, vop(3, dh), acc);
        acc = mfma4<4>(w4, vop(4, dh), acc);
        acc = mfma4<5>(w4, vop(5, dh), acc);
        acc = mfma4<6>(w4, vop(6, dh), acc);
        acc = mfma4<7>(w4, vop(7, dh), acc);
        acc = mfma4<8>(w4, vop(8, dh), acc);
        acc = mfma4<9>(w4, vop(9, dh), acc);
        acc = mfma4<10>(w4, vop(10, dh), acc);
        acc = mfma4<11>(w4, vop(11, dh), acc);
        acc = mfma4<12>(w4, vop(12, dh), acc);
        acc = mfma4<13>(w4, vop(13, dh), acc);
        acc = mfma4<14>(w4, vop(14, dh), acc);
        acc = mfma4<15>(w4, vop(15, dh), acc);
        st.acc[qd][dh] = acc;
    }
}

template <int D, int NQ>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
    constexpr int NS = D / 4;   // 4-dim k-steps of QK
    constexpr int NH = D / 64;  // 64-dim halves of P.V
    constexpr int RS = kHdr + D;
    __shared__ __attribute__((aligned(16))) uint16_t qs[NQ * NS * 4 * 4];
    __shared__ float wrec[kWavesPerGroup][kHeads * RS];

    const int split = blockIdx.x;
    const int kvh = blockIdx.y / a.head_groups;
    const int hgrp = blockIdx.y % a.head_groups;
    const int b = blockIdx.z;
    const int64_t bkv = (int64_t)b * a.L.Hkv + kvh;
    const int head0 = kvh * a.G + hgrp * kHeads;
    const int ng = min(kHeads, a.G - hgrp * kHeads);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int j = lane & 3, blk = lane >> 2;

    // query -> LDS as the B operand of the score MFMA: [qd][s][j][4 halves]
    for (int i = threadIdx.x; i < NQ * NS * 16; i += blockDim.x) {
        const int e = i & 3, jj = (i >> 2) & 3, sq = i >> 4;
        const int s = sq % NS, qd = sq / NS;
        const int h = 4 * qd + jj;
        qs[i] = h < ng ? a.q[((int64_t)b * a.Hq + head0 + h) * D + 4 * s + e] : (uint16_t)0;
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

    Lane<D, NQ> st;
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        st.m[qd] = -INFINITY;
        st.lsum[qd] = st.zsum[qd] = st.wsum[qd] = 0.f;
        st.mn[qd] = INFINITY;
        st.mx[qd] = -INFINITY;
        st.arg[qd] = INT_MAX;
#pragma unroll
        for (int dh = 0; dh < NH; dh++) st.acc[qd][dh] = fkv_f4{0.f, 0.f, 0.f, 0.f};
    }
    auto qop = [&](int qd, int s) {
        uint2 v;
        __builtin_memcpy(&v, qs + ((qd * NS + s) * 4 + j) * 4, 8);
        return __builtin_bit_cast(fkv_h4, v);
    };

    for (int k = k0 + wave; k < k1; k += kWavesPerGroup) {
        if (k >= nt_near && k < nt_near + nt_far) {
            // ------------------------------ far tile ------------------------------
            const int tile = k - nt_near;
            const uint8_t* kb = a.blob + a.L.far_k + (bkv * a.L.F_pad + (int64_t)tile * kTile) * D + lane * 16;
            const uint8_t* vb = a.blob + a.L.far_v + (bkv * a.L.F_pad + (int64_t)tile * kTile) * D / 2 + lane * 16;
            uint32_t kw[NS];     // dword s = dims 4s..4s+3 of token `lane`
            uint32_t vw[D / 8];  // nibble dwords of dim 64dh + lane
#pragma unroll
            for (int c = 0; c < D / 16; c++) {
                const uint4 x = *(const uint4*)(kb + c * 1024);
                kw[4 * c] = x.x; kw[4 * c + 1] = x.y; kw[4 * c + 2] = x.z; kw[4 * c + 3] = x.w;
            }
#pragma unroll
            for (int c = 0; c < D / 32; c++) {
                const uint4 x = *(const uint4*)(vb + c * 1024);
                vw[4 * c] = x.x; vw[4 * c + 1] = x.y; vw[4 * c + 2] = x.z; vw[4 * c + 3] = x.w;
            }
            const uint4 z4 = *(const uint4*)((const uint32_t*)(a.blob + a.L.far_sz) + bkv * a.L.F_pad +
                                             tile * kTile + 4 * blk);
            const uint32_t sz[4] = {z4.x, z4.y, z4.z, z4.w};
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) {
                fkv_f4 acc = fkv_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < NS; s++) acc = mfma4_local(e4m3x4(kw[s]), qop(qd, s), acc);
                float sc[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = tile * kTile + 4 * blk + e;
                    const float sv = acc[e] * a.inv_sqrt_d;
                    const bool ok = t < a.L.F;
                    sc[e] = ok ? sv : -INFINITY;
                    if (ok && sv > st.mx[qd]) { st.mx[qd] = sv; st.arg[qd] = t; }  // first index of the max
                }
                softmax_pv<D, NQ, true>(st, qd, sc, sz,
                                        [&](int g, int dh) { return int4x4(vw[dh * 8 + (g >> 1)], g & 1); });
            }
        } else {
            // ------------------- fp16 tile: near slots or decode rows -------------------
            const bool near = k < nt_near;
            const int tile = near ? k : k - nt_near - nt_far;
            const int count = near ? nv : a.n_dec;
            const int tk = tile * kTile + lane;  // this lane's token for the score operand
            fkv_f4 sacc[NQ];
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) sacc[qd] = fkv_f4{0.f, 0.f, 0.f, 0.f};
            const uint16_t* kb = (const uint16_t*)(a.blob + a.L.near_k) +
                                 (bkv * a.L.Na_pad + (int64_t)tile * kTile) * D + lane * 8;
            const uint16_t* kr = a.dec_k + (bkv * a.n_dec + (tk < count ? tk : 0)) * D;
#pragma unroll
            for (int cg = 0; cg < D / 32; cg++) {  // 4 chunks (8 steps) per round
                uint32_t kw[16];
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    uint4 x;
                    if (near) {
                        x = *(const uint4*)(kb + (cg * 4 + c) * 512);
                    } else {
                        x = tk < count ? *(const uint4*)(kr + (cg * 4 + c) * 8) : make_uint4(0, 0, 0, 0);
                    }
                    kw[4 * c] = x.x; kw[4 * c + 1] = x.y; kw[4 * c + 2] = x.z; kw[4 * c + 3] = x.w;
                }
#pragma unroll
                for (int qd = 0; qd < NQ; qd++)
#pragma unroll
                    for (int s = 0; s < 8; s++)
                        sacc[qd] = mfma4_local(h4_of(kw[2 * s], kw[2 * s + 1]), qop(qd, cg * 8 + s), sacc[qd]);
            }
            // values: 8-byte units x = dh*16 + g (4-token group g, dim 64dh + lane)
            uint32_t vw[D / 2];
            const uint16_t* vbn = (const uint16_t*)(a.blob + a.L.near_v) +
                                  (bkv * a.L.Na_pad + (int64_t)tile * kTile) * D + lane * 8;
#pragma unroll
            for (int c = 0; c < D / 8; c++) {
                uint4 x;
                if (near) {
                    x = *(const uint4*)(vbn + c * 512);
                } else {
                    uint16_t hv[8];
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        const int xi = 2 * c + u, g = xi % 16, dh = xi / 16;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const int tv = tile * kTile + 4 * g + e;
                            hv[4 * u + e] = tv < count ? a.dec_v[(bkv * a.n_dec + tv) * D + 64 * dh + lane] : (uint16_t)0;
                        }
                    }
                    x = make_uint4(hv[0] | ((uint32_t)hv[1] << 16), hv[2] | ((uint32_t)hv[3] << 16),
                                   hv[4] | ((uint32_t)hv[5] << 16), hv[6] | ((uint32_t)hv[7] << 16));
                }
                vw[4 * c] = x.x; vw[4 * c + 1] = x.y; vw[4 * c + 2] = x.z; vw[4 * c + 3] = x.w;
            }
            const uint32_t szd[4] = {0, 0, 0, 0};
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) {
                float sc[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = tile * kTile + 4 * blk + e;
                    const float sv = sacc[qd][e] * a.inv_sqrt_d;
                    const bool ok = t < count;
                    sc[e] = ok ? sv : -INFINITY;
                    if (ok) st.mn[qd] = fminf(st.mn[qd], sv);
                }
                softmax_pv<D, NQ, false>(st, qd, sc, szd, [&](int g, int dh) {
                    const int xi = dh * 16 + g;
                    return h4_of(vw[2 * xi], vw[2 * xi + 1]);
                });
            }
        }
    }

    // ---- per-head reduction over the 16 lanes (lane % 4 == head) ----
    float* wr = wrec[wave];
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        float l = st.lsum[qd], z = st.zsum[qd], ws = st.wsum[qd], mn = st.mn[qd], mx = st.mx[qd];
        int arg = st.arg[qd];
#pragma unroll
        for (int o = 4; o <= 32; o <<= 1) {
            l += wave_xor(l, o);
            z += wave_xor(z, o);
            ws += wave_xor(ws, o);
            mn = fminf(mn, wave_xor(mn, o));
            const float ox = wave_xor(mx, o);
            const int oa = wave_xor(arg, o);
            if (ox > mx || (ox == mx && oa < arg)) { mx = ox; arg = oa; }
        }
        z -= 23.5f * ws;  // remove the +16 INT4 decode offset and the 7.5 centring
        const float z0 = quad_bcast<0>(z), z1 = quad_bcast<1>(z), z2 = quad_bcast<2>(z), z3 = quad_bcast<3>(z);
        const int h = 4 * qd + j;
        if (lane < 4 && h < ng) {
            wr[h * RS + 0] = st.m[qd];
            wr[h * RS + 1] = l;
            wr[h * RS + 2] = mn;
            wr[h * RS + 3] = mx;
            wr[h * RS + 4] = __int_as_float(arg);
        }
        const float zz[4] = {z0, z1, z2, z3};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (4 * qd + i < ng) {
#pragma unroll
                for (int dh = 0; dh < NH; dh++) wr[(4 * qd + i) * RS + kHdr + 64 * dh + lane] = st.acc[qd][dh][i] + zz[i];
            }
        }
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

typedef void (*AttnKernel)(AttnArgs);

template <int D>
static AttnKernel pick_attn(int nq) {
    switch (nq) {
        case 1: return attn_kernel<D, 1>;
        case 2: return attn_kernel<D, 2>;
        case 3: return attn_kernel<D, 3>;
        default: return attn_kernel<D, 4>;
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
            hipLaunchKernelGGL(fkv::pack_near_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * L.Na_pad * (D / 16), blk)),
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
    const int nq = (ng_max + 3) / 4;
    fkv::AttnKernel k = L.D == 128 ? fkv::pick_attn<128>(nq) : fkv::pick_attn<64>(nq);
    hipLaunchKernelGGL(k, grid, block, 0, st, a);
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
