// Fused tier compression for gfx950: one pass over a layer's K and V builds
// the fp16 near tier (with zero headroom), the E4M3 far keys, the INT4
// per-token far values (+ fp16 scale / zero) and the fp16 far-row archive.
//
// Replaces CompressHandle::compress_layer (csrc/foveated_compress.cpp:95-201)
// and its three Metal kernels compress_foveal / compress_fp8 / compress_int4
// (csrc/kernels/foveated_compress.metal:76-205), whose outputs are
// reproduced bit-exactly:
//   * E4M3: re-biased exponent tested for saturation/underflow BEFORE
//     rounding, round-to-nearest-even on the 10->3 mantissa bits, a carry
//     into exponent 15 saturates to 0x7E (:39-66);
//   * INT4: fp32 row min/max, scale = max((max-min)/15, 1e-8) in fp32 with a
//     correctly rounded divide, codes = clamp(round((v-min)/scale), 0, 15)
//     with round-half-away-from-zero, even dim in the low nibble; the stored
//     scale and zero are the fp16 roundings (:153-205).
// Each row of D elements is owned by D/8 lanes (16 bytes of fp16 each).
#include <hip/hip_runtime.h>

#include <string>

#include "fkv_common.h"
#include "../../include/fkv.h"

namespace fkv {

struct CompressArgs {
    const void* k;
    const void* v;
    int dtype;
    int B, H, S;
    fkv_tiers tb;
    uint16_t* near_k;
    uint16_t* near_v;
    uint8_t* far_k;
    uint8_t* far_v;
    uint16_t* fvs;
    uint16_t* fvz;
    int32_t* near_valid;
    uint16_t* arc_k;
    uint16_t* arc_v;
};

__device__ inline uint8_t encode_e4m3(uint16_t bits) {
    const uint32_t sign = (uint32_t)(bits >> 15) << 7;
    const int ex = (bits >> 10) & 0x1f;
    const uint32_t man = bits & 0x3ffu;
    if (ex == 0) return (uint8_t)sign;
    if (ex == 31) return (uint8_t)(sign | 0x7eu);
    int e8 = ex - 8;
    if (e8 >= 15) return (uint8_t)(sign | 0x7eu);
    if (e8 <= 0) return (uint8_t)sign;
    uint32_t m3 = man >> 7;
    const bool up = ((man >> 6) & 1u) && ((man & 0x3fu) || (m3 & 1u));
    if (up) {
        m3++;
        if (m3 == 8) {
            m3 = 0;
            e8++;
            if (e8 >= 15) return (uint8_t)(sign | 0x7eu);
        }
    }
    return (uint8_t)(sign | ((uint32_t)e8 << 3) | m3);
}

// 8 consecutive elements as fp16 bits (astype(float16) semantics: RNE)
__device__ inline void load8(const void* base, int dtype, int64_t elem, uint16_t (&o)[8]) {
    if (dtype == FKV_F16) {
        const uint4 w = *(const uint4*)((const uint16_t*)base + elem);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[2 * i] = (uint16_t)(ws[i] & 0xffff);
            o[2 * i + 1] = (uint16_t)(ws[i] >> 16);
        }
    } else if (dtype == FKV_BF16) {
        const uint4 w = *(const uint4*)((const uint16_t*)base + elem);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[2 * i] = f2h(bf2f((uint16_t)(ws[i] & 0xffff)));
            o[2 * i + 1] = f2h(bf2f((uint16_t)(ws[i] >> 16)));
        }
    } else {
        const float4* p = (const float4*)((const float*)base + elem);
        const float4 a = p[0], b = p[1];
        const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = f2h(f[i]);
    }
}

__device__ inline uint4 pack8(const uint16_t (&x)[8]) {
    return make_uint4(x[0] | ((uint32_t)x[1] << 16), x[2] | ((uint32_t)x[3] << 16),
                      x[4] | ((uint32_t)x[5] << 16), x[6] | ((uint32_t)x[7] << 16));
}

// VG = 0: one INT4 scale / zero per token (the reference); VG = 32: one per
// 32-dim group (4 lanes), the same quantiser applied to every group.
template <int D, int VG>
__global__ __launch_bounds__(256) void compress_kernel(CompressArgs a) {
    constexpr int LPR = D / 8;       // lanes per row
    constexpr int RPB = 256 / LPR;   // rows per block
    const fkv_tiers& tb = a.tb;
    const int bh = blockIdx.y;
    const int r = blockIdx.x * RPB + threadIdx.x / LPR;
    const int sub = threadIdx.x % LPR;
    if (blockIdx.x == 0 && threadIdx.x == 0 && bh < a.H) a.near_valid[bh] = tb.r_actual;
    const int npad = tb.n_near_padded;
    const int F = tb.far_count;
    if (r >= a.S + tb.headroom) return;  // whole row group leaves together
    const uint4 zero4 = make_uint4(0, 0, 0, 0);
    if (r >= a.S) {  // headroom slot: zeros
        const int64_t o = ((int64_t)bh * npad + tb.r_actual + (r - a.S)) * D + sub * 8;
        *(uint4*)(a.near_k + o) = zero4;
        *(uint4*)(a.near_v + o) = zero4;
        return;
    }
    const int t = r;
    int slot = -1, f = -1;
    if (t < tb.n_sinks) slot = t;
    else if (t >= tb.near_mid_start && t < tb.mid_end) slot = tb.n_sinks + (t - tb.near_mid_start);
    else if (tb.window > 0 && t >= a.S - tb.window) slot = tb.n_sinks + tb.near_from_mid + (t - (a.S - tb.window));
    else if (t >= tb.mid_start && t < tb.near_mid_start) f = t - tb.mid_start;

    const int64_t src = ((int64_t)bh * a.S + t) * D + sub * 8;
    uint16_t kx[8], vx[8];
    load8(a.k, a.dtype, src, kx);
    load8(a.v, a.dtype, src, vx);
    if (slot >= 0) {
        const int64_t o = ((int64_t)bh * npad + slot) * D + sub * 8;
        *(uint4*)(a.near_k + o) = pack8(kx);
        *(uint4*)(a.near_v + o) = pack8(vx);
        return;
    }
    if (f < 0) return;  // unreachable: every position is near or far
    const int64_t fr = (int64_t)bh * F + f;
    // far K: E4M3 codes
    uint32_t c0 = 0, c1 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        c0 |= (uint32_t)encode_e4m3(kx[i]) << (8 * i);
        c1 |= (uint32_t)encode_e4m3(kx[4 + i]) << (8 * i);
    }
    *(uint2*)(a.far_k + fr * D + sub * 8) = make_uint2(c0, c1);
    // far V: INT4 per token (VG = 0) or per 32-dim group
    constexpr int RL = VG ? VG / 8 : LPR;  // lanes of one quantisation row
    float vf[8];
    float mn = INFINITY, mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        vf[i] = h2f(vx[i]);
        mn = fminf(mn, vf[i]);
        mx = fmaxf(mx, vf[i]);
    }
#pragma unroll
    for (int o = RL / 2; o >= 1; o >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, o, LPR));
        mx = fmaxf(mx, __shfl_xor(mx, o, LPR));
    }
    const float scale = fmaxf((mx - mn) / 15.0f, 1e-8f);
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float q = fminf(fmaxf(roundf((vf[i] - mn) / scale), 0.0f), 15.0f);
        packed |= (uint32_t)q << (4 * i);
    }
    *(uint32_t*)(a.far_v + fr * (D / 2) + sub * 4) = packed;
    if (sub % RL == 0) {
        const int64_t si = VG ? fr * (D / VG) + sub / RL : fr;
        a.fvs[si] = f2h(scale);
        a.fvz[si] = f2h(mn);
    }
    if (a.arc_k) *(uint4*)(a.arc_k + fr * D + sub * 8) = pack8(kx);
    if (a.arc_v) *(uint4*)(a.arc_v + fr * D + sub * 8) = pack8(vx);
}

}  // namespace fkv

extern "C" int fkv_compress_layer(const fkv_tier_config* cfg, const void* keys, const void* values,
                                  int32_t in_dtype, int32_t B, int32_t H, int32_t S, int32_t D,
                                  void* near_k, void* near_v, uint8_t* far_k, uint8_t* far_v,
                                  void* far_v_scale, void* far_v_zero, int32_t* near_valid,
                                  void* archive_k, void* archive_v, void* stream) {
    using fkv::set_error;
    if (!cfg) return set_error("fkv_compress_layer: cfg is NULL");
    if (B <= 0 || H <= 0 || S < 0) return set_error("fkv_compress_layer: bad shape");
    if (D != 64 && D != 128) return set_error("fkv_compress_layer: head dim must be 64 or 128, got " + std::to_string(D));
    if (in_dtype < FKV_F16 || in_dtype > FKV_F32) return set_error("fkv_compress_layer: unsupported dtype");
    if (cfg->v_group != 0 && cfg->v_group != 32)
        return set_error("fkv_compress_layer: v_group must be 0 (per token) or 32, got " + std::to_string(cfg->v_group));
    fkv_tiers tb;
    if (int rc = fkv_tier_boundaries(cfg, S, &tb)) return rc;
    if ((S > 0 && (!keys || !values)) || !near_k || !near_v || !near_valid ||
        (tb.far_count > 0 && (!far_k || !far_v || !far_v_scale || !far_v_zero)))
        return set_error("fkv_compress_layer: NULL output/input");
    fkv::CompressArgs a;
    a.k = keys;
    a.v = values;
    a.dtype = in_dtype;
    a.B = B;
    a.H = H;
    a.S = S;
    a.tb = tb;
    a.near_k = (uint16_t*)near_k;
    a.near_v = (uint16_t*)near_v;
    a.far_k = far_k;
    a.far_v = far_v;
    a.fvs = (uint16_t*)far_v_scale;
    a.fvz = (uint16_t*)far_v_zero;
    a.near_valid = near_valid;
    a.arc_k = (uint16_t*)archive_k;
    a.arc_v = (uint16_t*)archive_v;
    const int rows = S + tb.headroom;
    const int rpb = 256 / (D / 8);
    dim3 grid((unsigned)fkv::cdiv(rows > 0 ? rows : 1, rpb), (unsigned)(B * H));
    hipStream_t st = (hipStream_t)stream;
    const bool g32 = cfg->v_group == 32;
    void (*kern)(fkv::CompressArgs) = D == 128 ? (g32 ? fkv::compress_kernel<128, 32> : fkv::compress_kernel<128, 0>)
                                               : (g32 ? fkv::compress_kernel<64, 32> : fkv::compress_kernel<64, 0>);
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, a);
    return fkv::check_hip(hipGetLastError(), "compress_kernel launch");
}
