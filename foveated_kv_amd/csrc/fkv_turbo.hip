// TurboQuant far tier for gfx950: handle construction (blob packing), the
// per-call query rotation / sketch, and the compression kernels.
//
// Replaces the reference's TurboFoveatedHandle (csrc/foveated_attn.cpp:
// 280-491) and its Python compression (src/foveated_kv/turbo_quantize.py:
// 25-178).  The fused attention over a TurboQuant blob is attn_kernel<D,
// NQ, 1> in fkv_attn.hip; the record layout is described in fkv_attn.h.
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>

#include "fkv_attn.h"
#include "fkv_common.h"

namespace fkv {

// ---------------------------------------------------------------------------
// blob packing (csrc/foveated_attn.cpp:297-345 re-laid-out, fkv_attn.h)
// ---------------------------------------------------------------------------

__device__ inline uint8_t* tq_record(const BlobLayout& L, uint8_t* blob, int64_t bkv, int t) {
    return blob + L.far + far_rec_index(L, bkv, t / kTile) * (int64_t)L.far_rec;
}

// One thread per (bkv, far token, 32-dim word k): the three complemented key
// bit planes (index high bit, index low bit, QJL sign).
__global__ void tq_pack_k_kernel(const uint8_t* __restrict__ idx, const uint8_t* __restrict__ sgn, BlobLayout L,
                                 uint8_t* __restrict__ blob) {
    const int D = L.D, NK = D / 32;
    const int64_t n = (int64_t)L.B * L.Hkv * L.F_pad * NK;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int k = (int)(i % NK);
        const int64_t r = i / NK;
        const int t = (int)(r % L.F_pad);
        const int64_t bkv = r / L.F_pad;
        uint32_t wh = 0, wl = 0, ws = 0;
        if (t < L.F) {
            const uint8_t* ip = idx + (bkv * L.F + t) * (D / 4) + 8 * k;
            const uint8_t* sp = sgn + (bkv * L.F + t) * (D / 8) + 4 * k;
            for (int d = 0; d < 32; d++) {
                const int c = (ip[d >> 2] >> (2 * (d & 3))) & 3;
                const int sb = (sp[d >> 3] >> (d & 7)) & 1;
                const int bit = 15 - (d >> 1) + 16 * (d & 1);
                wh |= (uint32_t)((c >> 1) ^ 1) << bit;
                wl |= (uint32_t)((c & 1) ^ 1) << bit;
                ws |= (uint32_t)(sb ^ 1) << bit;
            }
        }
        uint8_t* rec = tq_record(L, blob, bkv, t);
        const int lt = t % kTile;
        ((uint32_t*)(rec + 0 * 8 * D + lt * (D / 8)))[k] = wh;
        ((uint32_t*)(rec + 1 * 8 * D + lt * (D / 8)))[k] = wl;
        ((uint32_t*)(rec + 2 * 8 * D + lt * (D / 8)))[k] = ws;
    }
}

// One thread per (bkv, tile, 64-dim half dh, lane l): the lane's four value
// plane dwords for dim 64dh + l.
__global__ void tq_pack_v_kernel(const uint8_t* __restrict__ vp, BlobLayout L, uint8_t* __restrict__ blob) {
    const int D = L.D, NT = L.F_pad / kTile, NHALF = D / 64;
    const int64_t n = (int64_t)L.B * L.Hkv * NT * NHALF * 64;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int l = (int)(i % 64);
        int64_t r = i / 64;
        const int dh = (int)(r % NHALF);
        r /= NHALF;
        const int tile = (int)(r % NT);
        const int64_t bkv = r / NT;
        const int d = 64 * dh + l, half = l >> 5;
        uint32_t w[4] = {0u, 0u, 0u, 0u};  // hi own, hi other, lo own, lo other
        for (int o = 0; o < 2; o++) {
            const int base = 32 * (o ? 1 - half : half);
            for (int jj = 0; jj < 32; jj++) {
                const int t = tile * kTile + base + jj;
                int c = 3;  // padding tokens: +1 bits (their weights are zero)
                if (t < L.F) c = (vp[(bkv * L.F + t) * (D / 4) + d / 4] >> (2 * (d & 3))) & 3;
                const int bit = 15 - (jj >> 1) + 16 * (jj & 1);
                w[o] |= (uint32_t)((c >> 1) ^ 1) << bit;
                w[2 + o] |= (uint32_t)((c & 1) ^ 1) << bit;
            }
        }
        uint32_t* dst = (uint32_t*)(blob + L.far + far_rec_index(L, bkv, tile) * (int64_t)L.far_rec +
                                    tq_vp_section(D) + dh * 1024 + l * 16);
        dst[0] = w[0];
        dst[1] = w[1];
        dst[2] = w[2];
        dst[3] = w[3];
    }
}

// One thread per (bkv, far token): value group scales and norm | gamma.
__global__ void tq_pack_sn_kernel(const void* __restrict__ vscale, const void* __restrict__ knorm,
                                  const void* __restrict__ kgamma, int dtype, BlobLayout L,
                                  uint8_t* __restrict__ blob) {
    const int D = L.D, NG = D / 32;
    const int64_t n = (int64_t)L.B * L.Hkv * L.F_pad;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(i % L.F_pad);
        const int64_t bkv = i / L.F_pad;
        uint8_t* rec = tq_record(L, blob, bkv, t);
        const int lt = t % kTile;
        uint16_t* sc = (uint16_t*)(rec + tq_sc_section(D));
        const int64_t tok = bkv * L.F + t;
        for (int g = 0; g < NG; g++)
            sc[tq_sc_index(D, lt / 4, g % 2, lt % 4, g / 2)] = t < L.F ? load_as_f16(vscale, tok * NG + g, dtype)
                                                                      : (uint16_t)0;
        uint32_t w = 0;
        if (t < L.F) w = (uint32_t)load_as_f16(knorm, tok, dtype) | ((uint32_t)load_as_f16(kgamma, tok, dtype) << 16);
        ((uint32_t*)(rec + tq_ng_section(D)))[lt] = w;
    }
}

// out[j][i] = in[i][j] for a (D, D) fp32 matrix.
// Pi and S -> the rotation MFMAs' fp16 operands (tq_rot_index).
__global__ void rot_operand_kernel(const float* __restrict__ Pi, const float* __restrict__ S,
                                   uint16_t* __restrict__ rot, int D) {
    const int64_t n = 2 * (int64_t)D * D;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int mat = (int)(e / ((int64_t)D * D)), i = (int)(e / D % D), j = (int)(e % D);
        rot[tq_rot_index(D, mat, i, j)] = f2h((mat ? S : Pi)[(int64_t)i * D + j]);
    }
}

__global__ void transpose_kernel(const float* __restrict__ in, float* __restrict__ out, int D) {
    const int64_t n = (int64_t)D * D;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / D), c = (int)(i % D);
        out[(int64_t)c * D + r] = in[i];
    }
}

// ---------------------------------------------------------------------------
// per-call query preparation (csrc/foveated_attn.cpp:415-421)
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// compression (src/foveated_kv/turbo_quantize.py:25-91, 139-178), fp32
// ---------------------------------------------------------------------------

constexpr int kTqTok = 32;  // tokens per workgroup of the key compressor

// One workgroup (256 threads) per 32 tokens.  Thread (dim i, token group)
// accumulates 32 / (256 / D) tokens' outputs for dim i; the matrix rows are
// read once per workgroup (coalesced across i), the token rows from LDS.
//   n = |k|; y = (k / max(n, 1e-8)) Pi^T; idx = [y >= b0] + [y >= b1] + [y >= b2]
//   r = k - n * (cb[idx] Pi); gamma = |r|; sign = (r S^T >= 0)
template <int D>
__global__ __launch_bounds__(256) void tq_compress_keys_kernel(const void* __restrict__ keys, int dtype, int64_t n_tok,
                                                               const float* __restrict__ PiT,
                                                               const float* __restrict__ Pi,
                                                               const float* __restrict__ ST, float4 cbv, float4 bdv,
                                                               uint8_t* __restrict__ out_idx,
                                                               uint8_t* __restrict__ out_sgn,
                                                               uint16_t* __restrict__ out_norm,
                                                               uint16_t* __restrict__ out_gamma) {
    constexpr int TG = 256 / D, TPT = kTqTok / TG;  // token groups, tokens per thread
    __shared__ float kf[kTqTok][D];   // k, later r
    __shared__ float kn[kTqTok][D];   // k / max(n, 1e-8), later cb[idx]
    __shared__ uint8_t codes[kTqTok][D];
    __shared__ float nrm[kTqTok], gam[kTqTok];
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int i = tid % D, tg = tid / D;
    const int64_t t0 = (int64_t)blockIdx.x * kTqTok;
    const float cb[4] = {cbv.x, cbv.y, cbv.z, cbv.w};
    for (int e = tid; e < kTqTok * D; e += 256) {
        const int tt = e / D, d = e % D;
        const int64_t t = t0 + tt;
        kf[tt][d] = t < n_tok ? h2f(load_as_f16(keys, t * D + d, dtype)) : 0.f;
    }
    __syncthreads();
    for (int tt = wave; tt < kTqTok; tt += 4) {
        float ss = 0.f;
        for (int d = lane; d < D; d += 64) ss += kf[tt][d] * kf[tt][d];
        ss = wave_sum(ss);
        if (lane == 0) nrm[tt] = sqrtf(ss);
    }
    __syncthreads();
    for (int e = tid; e < kTqTok * D; e += 256) {
        const int tt = e / D, d = e % D;
        kn[tt][d] = kf[tt][d] / fmaxf(nrm[tt], 1e-8f);
    }
    __syncthreads();
    float acc[TPT];
#pragma unroll
    for (int u = 0; u < TPT; u++) acc[u] = 0.f;
    for (int j = 0; j < D; j++) {
        const float m = PiT[j * D + i];
#pragma unroll
        for (int u = 0; u < TPT; u++) acc[u] = fmaf(kn[tg * TPT + u][j], m, acc[u]);
    }
    __syncthreads();  // every y is computed: kn may be overwritten with the centroids
#pragma unroll
    for (int u = 0; u < TPT; u++) {
        const float y = acc[u];
        const int c = (y >= bdv.x) + (y >= bdv.y) + (y >= bdv.z);
        codes[tg * TPT + u][i] = (uint8_t)c;
        kn[tg * TPT + u][i] = cb[c];
        acc[u] = 0.f;
    }
    __syncthreads();
    for (int j = 0; j < D; j++) {  // (cb[idx] Pi)_i = sum_j cb[idx_j] Pi[j][i]
        const float m = Pi[j * D + i];
#pragma unroll
        for (int u = 0; u < TPT; u++) acc[u] = fmaf(kn[tg * TPT + u][j], m, acc[u]);
    }
#pragma unroll
    for (int u = 0; u < TPT; u++) {
        const int tt = tg * TPT + u;
        kf[tt][i] = kf[tt][i] - nrm[tt] * acc[u];  // residual
        acc[u] = 0.f;
    }
    __syncthreads();
    for (int tt = wave; tt < kTqTok; tt += 4) {
        float ss = 0.f;
        for (int d = lane; d < D; d += 64) ss += kf[tt][d] * kf[tt][d];
        ss = wave_sum(ss);
        if (lane == 0) gam[tt] = sqrtf(ss);
    }
    for (int j = 0; j < D; j++) {  // (r S^T)_i = sum_j r_j ST[j][i]
        const float m = ST[j * D + i];
#pragma unroll
        for (int u = 0; u < TPT; u++) acc[u] = fmaf(kf[tg * TPT + u][j], m, acc[u]);
    }
    __syncthreads();  // residual reads done, gamma written
#pragma unroll
    for (int u = 0; u < TPT; u++) kn[tg * TPT + u][i] = acc[u] >= 0.f ? 1.f : 0.f;
    __syncthreads();
    for (int e = tid; e < kTqTok * (D / 4); e += 256) {
        const int tt = e / (D / 4), by = e % (D / 4);
        const int64_t t = t0 + tt;
        if (t >= n_tok) continue;
        const uint8_t* c = &codes[tt][4 * by];
        out_idx[t * (D / 4) + by] = (uint8_t)(c[0] | (c[1] << 2) | (c[2] << 4) | (c[3] << 6));
        if (by < D / 8) {
            uint32_t b = 0;
            for (int k = 0; k < 8; k++) b |= (kn[tt][8 * by + k] != 0.f ? 1u : 0u) << k;
            out_sgn[t * (D / 8) + by] = (uint8_t)b;
        }
        if (by == 0) {
            out_norm[t] = f2h(nrm[tt]);
            out_gamma[t] = f2h(gam[tt]);
        }
    }
}

// One thread per (token, 32-dim group): scale = max(max|v|, 1e-8), code =
// clip(rint((v / scale + 1) * 1.5), 0, 3) (round half to even, as mx.round).
__global__ void tq_compress_values_kernel(const void* __restrict__ vals, int dtype, int64_t n_groups,
                                          uint8_t* __restrict__ out_packed, uint16_t* __restrict__ out_scale) {
    for (int64_t gi = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; gi < n_groups;
         gi += (int64_t)gridDim.x * blockDim.x) {
        float v[32];
        float mx = 0.f;
#pragma unroll
        for (int k = 0; k < 32; k++) {
            v[k] = h2f(load_as_f16(vals, gi * 32 + k, dtype));
            mx = fmaxf(mx, fabsf(v[k]));
        }
        const float sc = fmaxf(mx, 1e-8f);
        uint32_t w[2] = {0u, 0u};
#pragma unroll
        for (int k = 0; k < 32; k++) {
            const float x = (v[k] / sc + 1.0f) * 1.5f;
            const float r = fminf(fmaxf(rintf(x), 0.f), 3.f);
            w[k >> 4] |= (uint32_t)r << (2 * (k & 15));
        }
        uint2* dst = (uint2*)(out_packed + gi * 8);
        *dst = make_uint2(w[0], w[1]);
        out_scale[gi] = f2h(sc);
    }
}

}  // namespace fkv

using fkv::check_hip;
using fkv::set_error;

extern "C" {

int fkv_turbo_create(fkv_attn** out, int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F,
                     const void* near_k, const void* near_v, int32_t near_dtype, const uint8_t* k_idx,
                     const uint8_t* k_signs, const void* k_norm, const void* k_gamma, const uint8_t* v_packed,
                     const void* v_scale, int32_t nz_dtype, const int32_t* near_valid, const float* Pi,
                     const float* S, const float* centroids, float spike_margin, void* stream) {
    if (!out) return set_error("fkv_turbo_create: out is NULL");
    *out = nullptr;
    if (B <= 0 || Hkv <= 0 || Na < 0 || F < 0)
        return set_error("fkv_turbo_create: bad shape B=" + std::to_string(B) + " Hkv=" + std::to_string(Hkv) +
                         " Na=" + std::to_string(Na) + " F=" + std::to_string(F));
    if (D != 64 && D != 128) return set_error("fkv_turbo_create: head dim must be 64 or 128, got " + std::to_string(D));
    if (near_dtype < FKV_F16 || near_dtype > FKV_F32 || nz_dtype < FKV_F16 || nz_dtype > FKV_F32)
        return set_error("fkv_turbo_create: unsupported dtype");
    if ((Na > 0 && (!near_k || !near_v)) ||
        (F > 0 && (!k_idx || !k_signs || !k_norm || !k_gamma || !v_packed || !v_scale)) || !near_valid || !Pi ||
        !S || !centroids)
        return set_error("fkv_turbo_create: NULL array");
    hipStream_t st = (hipStream_t)stream;
    fkv_attn* h = new fkv_attn();
    int rc = fkv::attn_begin(h, B, Hkv, D, Na, F, 1, near_k, near_v, near_dtype, near_valid, spike_margin, st);
    if (!rc) rc = check_hip(hipMalloc(&h->tq.rot, (size_t)4 * D * D), "hipMalloc(rotation operands)");
    float cb[4] = {0.f, 0.f, 0.f, 0.f};
    if (!rc) {
        const int blk = 256;
        const fkv::BlobLayout L = h->L;
        hipLaunchKernelGGL(fkv::rot_operand_kernel, dim3(fkv::grid_for(2 * (int64_t)D * D, blk)), dim3(blk), 0, st,
                           Pi, S, h->tq.rot, D);
        if (F > 0) {
            hipLaunchKernelGGL(fkv::tq_pack_k_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * L.F_pad * (D / 32), blk)),
                               dim3(blk), 0, st, k_idx, k_signs, L, h->blob);
            hipLaunchKernelGGL(fkv::tq_pack_v_kernel,
                               dim3(fkv::grid_for((int64_t)B * Hkv * (L.F_pad / fkv::kTile) * D, blk)), dim3(blk), 0,
                               st, v_packed, L, h->blob);
            hipLaunchKernelGGL(fkv::tq_pack_sn_kernel, dim3(fkv::grid_for((int64_t)B * Hkv * L.F_pad, blk)),
                               dim3(blk), 0, st, v_scale, k_norm, k_gamma, nz_dtype, L, h->blob);
        }
        rc = check_hip(hipGetLastError(), "turbo pack kernels");
    }
    if (!rc) rc = check_hip(hipMemcpyAsync(cb, centroids, sizeof(cb), hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    if (!rc) rc = fkv::attn_finish(h, st);
    if (!rc) {
        // centroid(c) = alpha + beta*sh + gamma*sl + delta*sh*sl, sh/sl = +-1 bits of c
        const double c0 = cb[0], c1 = cb[1], c2 = cb[2], c3 = cb[3];
        h->tq.alpha = (float)((c0 + c1 + c2 + c3) / 4);
        h->tq.beta = (float)((c2 + c3 - c0 - c1) / 4);
        h->tq.gamma = (float)((c1 + c3 - c0 - c2) / 4);
        h->tq.delta = (float)((c0 + c3 - c1 - c2) / 4);
        // value levels {-1, -0.333333, 0.333333, 1} (csrc/kernels/foveated_attn.metal:529)
        const double l0 = -1.0, l1 = (double)-0.333333f, l2 = (double)0.333333f, l3 = 1.0;
        h->tq.lvh = (float)((l2 + l3 - l0 - l1) / 4);
        h->tq.lvl = (float)((l1 + l3 - l0 - l2) / 4);
        // the kernel expands the high-bit value plane to +-2 against
        // weights scaled by lvl (one weight for both planes)
        if (std::fabs(h->tq.lvh - 2.0 * h->tq.lvl) > 2e-6 * h->tq.lvh)
            rc = fkv::set_error("fkv_turbo_create: value levels with lvh != 2 lvl (internal error)");
    }
    if (rc) {
        fkv_attn_destroy(h);
        return rc;
    }
    *out = h;
    return FKV_OK;
}

int fkv_turbo_compress_keys(const void* keys, int32_t dtype, int64_t n_tokens, int32_t D, const float* Pi,
                            const float* S, const float* centroids, const float* boundaries, uint8_t* out_idx,
                            uint8_t* out_signs, void* out_norm, void* out_gamma, void* stream) {
    if (D != 64 && D != 128) return set_error("fkv_turbo_compress_keys: head dim must be 64 or 128");
    if (dtype < FKV_F16 || dtype > FKV_F32) return set_error("fkv_turbo_compress_keys: unsupported dtype");
    if (n_tokens < 0) return set_error("fkv_turbo_compress_keys: negative token count");
    if (n_tokens == 0) return FKV_OK;
    if (!keys || !Pi || !S || !centroids || !boundaries || !out_idx || !out_signs || !out_norm || !out_gamma)
        return set_error("fkv_turbo_compress_keys: NULL argument");
    hipStream_t st = (hipStream_t)stream;
    float cbh[8];
    int rc = check_hip(hipMemcpyAsync(cbh, centroids, 4 * sizeof(float), hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    if (!rc) rc = check_hip(hipMemcpyAsync(cbh + 4, boundaries, 3 * sizeof(float), hipMemcpyDeviceToHost, st),
                            "hipMemcpyAsync");
    if (!rc) rc = check_hip(hipStreamSynchronize(st), "hipStreamSynchronize");
    float* PiT = nullptr;
    float* ST = nullptr;
    const size_t mat = (size_t)D * D * sizeof(float);
    if (!rc) rc = check_hip(hipMallocAsync((void**)&PiT, mat, st), "hipMallocAsync");
    if (!rc) rc = check_hip(hipMallocAsync((void**)&ST, mat, st), "hipMallocAsync");
    if (!rc) {
        hipLaunchKernelGGL(fkv::transpose_kernel, dim3(fkv::grid_for((int64_t)D * D, 256)), dim3(256), 0, st, Pi, PiT, D);
        hipLaunchKernelGGL(fkv::transpose_kernel, dim3(fkv::grid_for((int64_t)D * D, 256)), dim3(256), 0, st, S, ST, D);
        const float4 cbv = make_float4(cbh[0], cbh[1], cbh[2], cbh[3]);
        const float4 bdv = make_float4(cbh[4], cbh[5], cbh[6], 0.f);
        const dim3 grid((unsigned)fkv::cdiv(n_tokens, fkv::kTqTok));
        if (D == 128)
            hipLaunchKernelGGL(fkv::tq_compress_keys_kernel<128>, grid, dim3(256), 0, st, keys, dtype, n_tokens, PiT, Pi,
                               ST, cbv, bdv, out_idx, out_signs, (uint16_t*)out_norm, (uint16_t*)out_gamma);
        else
            hipLaunchKernelGGL(fkv::tq_compress_keys_kernel<64>, grid, dim3(256), 0, st, keys, dtype, n_tokens, PiT, Pi,
                               ST, cbv, bdv, out_idx, out_signs, (uint16_t*)out_norm, (uint16_t*)out_gamma);
        rc = check_hip(hipGetLastError(), "tq_compress_keys_kernel launch");
    }
    if (PiT) (void)hipFreeAsync(PiT, st);
    if (ST) (void)hipFreeAsync(ST, st);
    return rc;
}

int fkv_turbo_compress_values(const void* values, int32_t dtype, int64_t n_tokens, int32_t D, uint8_t* out_packed,
                              void* out_scale, void* stream) {
    if (D <= 0 || D % 32 != 0) return set_error("fkv_turbo_compress_values: head dim must be a multiple of 32");
    if (dtype < FKV_F16 || dtype > FKV_F32) return set_error("fkv_turbo_compress_values: unsupported dtype");
    if (n_tokens < 0) return set_error("fkv_turbo_compress_values: negative token count");
    if (n_tokens == 0) return FKV_OK;
    if (!values || !out_packed || !out_scale) return set_error("fkv_turbo_compress_values: NULL argument");
    const int64_t ng = n_tokens * (D / 32);
    hipLaunchKernelGGL(fkv::tq_compress_values_kernel, dim3(fkv::grid_for(ng, 256)), dim3(256), 0,
                       (hipStream_t)stream, values, dtype, ng, out_packed, (uint16_t*)out_scale);
    return check_hip(hipGetLastError(), "tq_compress_values_kernel launch");
}

}  // extern "C"
