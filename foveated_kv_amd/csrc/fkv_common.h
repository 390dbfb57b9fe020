// Shared device/host definitions for the FoveatedKV gfx950 library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

typedef _Float16 fkv_h2 __attribute__((ext_vector_type(2)));
typedef float fkv_f2 __attribute__((ext_vector_type(2)));

namespace fkv {

constexpr int kWave = 64;          // CDNA wavefront
constexpr int kTile = 64;          // tokens per wave iteration (one per lane)
constexpr int kWavesPerGroup = 4;  // waves per workgroup of the attention kernel

// Sets the thread-local error string returned by fkv_last_error().
int set_error(const std::string& msg);
int check_hip(hipError_t e, const char* what);

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ inline int64_t round_up(int64_t a, int64_t b) { return cdiv(a, b) * b; }

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

__device__ inline float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ inline uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ inline float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ inline fkv_h2 as_h2(uint32_t u) { return __builtin_bit_cast(fkv_h2, u); }
__device__ inline uint32_t as_u32(fkv_h2 h) { return __builtin_bit_cast(uint32_t, h); }

// acc + a.x*b.x + a.y*b.y with fp32 accumulation (v_dot2_f32_f16).
__device__ inline float dot2(fkv_h2 a, fkv_h2 b, float acc) {
    return __builtin_amdgcn_fdot2(a, b, acc, false);
}

// Two E4M3 codes (selected 16-bit word of src) -> two fp16 values, exact for
// every normal E4M3 value (v_cvt_scalef32_pk_f16_fp8 with unit scale).
__device__ inline fkv_h2 e4m3x2_to_h2(uint32_t src, bool hi_word) {
    return hi_word ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(src, 1.0f, true)
                   : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(src, 1.0f, false);
}

template <typename T>
__device__ inline T wave_xor(T v, int mask) {
    return __shfl_xor(v, mask, kWave);
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, wave_xor(v, o));
    return v;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += wave_xor(v, o);
    return v;
}

__device__ inline float wave_min(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fminf(v, wave_xor(v, o));
    return v;
}

// Wave-wide (max, first index) reduction: larger value wins, ties go to the
// smaller index.  Lanes with no candidate hold (-inf, INT_MAX).
__device__ inline void wave_argmax(float& v, int& idx) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        float ov = wave_xor(v, o);
        int oi = wave_xor(idx, o);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
}

}  // namespace fkv
