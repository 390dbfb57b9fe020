// Device code of the fused two-tier decode attention: the operand
// helpers, the per-tile computations and the attn_kernel template.  Included
// by the translation units that instantiate the kernels: fkv_attn.hip
// (TurboQuant rows and the separate merge launch), fkv_attn_q1.hip (fp8 and
// group-32 rows of one head quad) and fkv_attn_qn.hip (rows of 2-4 head
// quads); each is compiled with the instruction scheduling that measured
// fastest for its kernels.  The layout and the algorithm are described at
// the top of fkv_attn.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <type_traits>

#include "fkv_attn.h"
#include "fkv_common.h"

typedef _Float16 fkv_h4 __attribute__((ext_vector_type(4)));
typedef float fkv_f4 __attribute__((ext_vector_type(4)));

namespace fkv {

// Phase stamps (a build with -DFKV_PHASE_STAMPS only; the default build
// compiles them out): per workgroup of an attention launch, thread 0 / each
// wave's lane 0 stores the 100 MHz constant clock (s_memrealtime) at fixed
// points into a.stamps[64 * linear workgroup index + slot] (a device array
// of fkv_attn.hip), and the XCD id into slot 63; fkv_phase_stamps copies
// them out.  Slots: 0 entry, 1 prologue done (query landed, stream about to
// start), 2 + w wave w's stream and decode tiles done, 20 records published
// (before the arrival), 21 arrival counted, 22 the last split's merge done.
constexpr int kStampSlots = 64, kStampWGs = 8192;
#ifdef FKV_PHASE_STAMPS
#define FKV_STAMP_AT(cond, slot)                                                                             \
    do {                                                                                                    \
        if (cond) {                                                                                         \
            const int wg_ = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;                 \
            if (wg_ < kStampWGs) a.stamps[kStampSlots * wg_ + (slot)] = __builtin_amdgcn_s_memrealtime();  \
        }                                                                                                   \
    } while (0)
#else
#define FKV_STAMP_AT(cond, slot) \
    do {                         \
    } while (0)
#endif


// ---------------------------------------------------------------------------
// Attention kernel
// ---------------------------------------------------------------------------

constexpr int kHeads = 16;  // query heads per workgroup row: up to 4 quads of 4
constexpr int kSmallGrid = 64;  // fewer workgroups than this: rows of 4 query heads
// record header: m, l, min_near, max_far, first argmax, 3 unused (records
// of kHdr + D floats stay 16-byte aligned for the direct merge's loads)
constexpr int kHdr = 8;
constexpr int kMaxSplits = 64;

// Waves per workgroup of the attention kernel (one workgroup per CU): 8 for
// TurboQuant rows of one head quad at D = 128 -- two waves per SIMD, whose
// far tile is bound by dependent VALU / MFMA chains that the second wave
// overlaps (8 KB ring units, registers within 256) while the query rotation
// is still loaded and computed once per CU -- and 4 elsewhere.
__host__ __device__ constexpr int attn_waves(int D, int NQ, int fmt) {
    return fmt == 1 && D == 128 && NQ == 1 ? 8 : kWavesPerGroup;
}

struct AttnArgs {
    const uint8_t* blob;
    BlobLayout L;
    const uint16_t* q;      // (B, Hq, D) fp16
    const uint16_t* dec_k;  // (B, Hkv, dec_stride, D) fp16 rows, the first n_dec valid
    const uint16_t* dec_v;
    int n_dec;
    int dec_stride;
    const int32_t* n_dec_dev;  // when set, n_dec is read here (clamped to [0, dec_stride])
    int Hq;
    int G;            // query heads per kv head
    int head_groups;  // workgroup rows per kv head (ceil(G / hpg))
    int hpg;          // query heads per workgroup row (4 or kHeads)
    int num_splits;
    float spike_margin;
    float inv_sqrt_d;
    uint16_t* out;  // (B, Hq, D) fp16
    int32_t* flags;
    int32_t* tokens;
    float* ws;      // split partials: [row][split][ng][kHdr + D]
    int* arrive;    // [row] split arrival counters (zero between calls)
    // XCD-local merge watch (xcd_mod != 0): a flag the merging workgroups
    // raise when a split record of their row came from another XCD
    uint32_t* xcd_watch;
    int near_plan;  // expected near tiles per row (balances the far split)
    int dec_wave0;  // the wave that takes decode tile 0
    int wave_recs;  // split records per split: 4 (one per wave) or 1 (merged in LDS)
    // XCD-local split merge (see the merge section): the XCD count X of the
    // dispatch rule, 0 where the merge goes through memory instead
    int xcd_mod;
    // TurboQuant far tier (fmt 1)
    const uint16_t* tq_rot; // Pi, S as rotation MFMA operands (tq_rot_index)
    float tq_alpha;         // centroid constant term (0 for a symmetric codebook)
    float tq_beta, tq_gamma, tq_delta;  // centroid coefficients (TurboConsts)
    float tq_qjl;           // 1.2533141 / D
    float tq_lvh, tq_lvl;   // value level coefficients
    // Extensions (read by the EXT kernels only; last, so the fields above
    // keep their kernel-argument offsets).  Top-K spike selection (spike_k >
    // 1, else NULL): every far tile's maximum score per query head, (B*Hq,
    // tmax_stride = far tiles) fp32, and each head's spike threshold
    // min_near + margin, (B*Hq) fp32; the top-K candidates kernel reads
    // both after the launch
    float* tmax;
    int tmax_stride;
    float* thr;
    // per-head fp8 key scales, (B*Hkv) fp32 in the blob; NULL for a handle
    // whose keys are unscaled (no load then: the scale is 1)
    const float* kscale;
#ifdef FKV_PHASE_STAMPS
    unsigned long long* stamps;  // kStampSlots per workgroup (fkv_phase_stamps)
#endif
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
// The mask and the exponent bits are held in registers (empty asm, no
// instruction): gfx9 VOP3 takes no literal, so with folded constants each
// half costs a shift, an AND and an OR instead of a shift and one
// v_and_or_b32.
__device__ inline fkv_h4 int4x4(uint32_t w, int bp) {
    uint32_t m = 0x03C003C0u, e = 0x4C004C00u;
    asm("" : "+s"(m));
    asm("" : "+v"(e));
    const uint32_t a = bp ? (w >> 2) : (w << 6);
    const uint32_t b = bp ? (w >> 6) : (w << 2);
    return h4_of((a & m) | e, (b & m) | e);
}

// int4x4 of two INT4 dwords at once: w = (w1 << 32) | w0, where w0 holds
// 4-token groups 2u, 2u + 1 and w1 groups 2u + 2, 2u + 3.  One 64-bit shift
// serves both dwords: the bits a shift carries across the dword boundary
// land at bits 0-5 (left shifts) or 26-31 (right shifts), outside the mask
// (bits 6-9, 22-25).  The shift amounts are opaque (empty asm on scalar
// registers), so the compiler keeps one v_lshlrev_b64 / v_lshrrev_b64
// (issued at the rate of the 32-bit shifts) instead of splitting each into
// two 32-bit ones.  o[i] = int4x4(w_{i / 2}, i % 2).
__device__ inline void int4x4_pair(uint64_t w, fkv_h4 (&o)[4]) {
    uint32_t m = 0x03C003C0u, e = 0x4C004C00u, n2 = 2, n6 = 6;
    asm("" : "+s"(m));
    asm("" : "+v"(e));
    asm("" : "+s"(n2));
    asm("" : "+s"(n6));
    const uint64_t a0 = w << n6, b0 = w << n2, a1 = w >> n2, b1 = w >> n6;
    o[0] = h4_of(((uint32_t)a0 & m) | e, ((uint32_t)b0 & m) | e);
    o[1] = h4_of(((uint32_t)a1 & m) | e, ((uint32_t)b1 & m) | e);
    o[2] = h4_of(((uint32_t)(a0 >> 32) & m) | e, ((uint32_t)(b0 >> 32) & m) | e);
    o[3] = h4_of(((uint32_t)(a1 >> 32) & m) | e, ((uint32_t)(b1 >> 32) & m) | e);
}

// broadcast lane i of each lane quad (DPP quad_perm)
template <int I>
__device__ inline float quad_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), I * 0x55, 0xF, 0xF, false));
}

// Cross-lane reductions over the 16 lanes that share lane % 4 (one head of
// a quad) without LDS permutes: DPP row rotations by 4 and 8 lanes cover a
// row of 16, v_permlane16_swap / v_permlane32_swap the other rows.  A swap
// returns (this lane's new vdst, new vsrc); with vdst = vsrc = v the pair is
// {v[l], v[l ^ 16]} (or ^ 32) in an order that depends on the lane, so only
// symmetric combinations of the two are taken.
template <int N>
__device__ inline uint32_t row_ror(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x120 + N, 0xF, 0xF, false);
}
struct LanePair {
    uint32_t a, b;
};
__device__ inline LanePair swap16(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return {r[0], r[1]};
}
__device__ inline LanePair swap32(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return {r[0], r[1]};
}
// max over the lanes l' = l (mod 4) of the wave
__device__ inline float head_max(float v) {
    v = fmaxf(v, __uint_as_float(row_ror<4>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(row_ror<8>(__float_as_uint(v))));
    LanePair p = swap16(__float_as_uint(v));
    v = fmaxf(__uint_as_float(p.a), __uint_as_float(p.b));
    p = swap32(__float_as_uint(v));
    return fmaxf(__uint_as_float(p.a), __uint_as_float(p.b));
}
__device__ inline float head_min(float v) {
    v = fminf(v, __uint_as_float(row_ror<4>(__float_as_uint(v))));
    v = fminf(v, __uint_as_float(row_ror<8>(__float_as_uint(v))));
    LanePair p = swap16(__float_as_uint(v));
    v = fminf(__uint_as_float(p.a), __uint_as_float(p.b));
    p = swap32(__float_as_uint(v));
    return fminf(__uint_as_float(p.a), __uint_as_float(p.b));
}
// sum over the lanes l' = l (mod 4) of this lane's 32-lane half (WHOLE = false)
// or of the whole wave
template <bool WHOLE>
__device__ inline float head_sum(float v) {
    v += __uint_as_float(row_ror<4>(__float_as_uint(v)));
    v += __uint_as_float(row_ror<8>(__float_as_uint(v)));
    LanePair p = swap16(__float_as_uint(v));
    v = __uint_as_float(p.a) + __uint_as_float(p.b);
    if (WHOLE) {
        p = swap32(__float_as_uint(v));
        v = __uint_as_float(p.a) + __uint_as_float(p.b);
    }
    return v;
}
// (max, first index of the max) over the lanes l' = l (mod 4)
__device__ inline void pick_max(float& mx, int& arg, float ox, int oa) {
    // bitwise, not short-circuit: three compares and two selects (a || / &&
    // here compiles to branches around each compare)
    const bool take = (ox > mx) | ((ox == mx) & (oa < arg));
    mx = take ? ox : mx;
    arg = take ? oa : arg;
}
__device__ inline void head_argmax(float& mx, int& arg) {
    pick_max(mx, arg, __uint_as_float(row_ror<4>(__float_as_uint(mx))), (int)row_ror<4>((uint32_t)arg));
    pick_max(mx, arg, __uint_as_float(row_ror<8>(__float_as_uint(mx))), (int)row_ror<8>((uint32_t)arg));
    LanePair pm = swap16(__float_as_uint(mx)), pa = swap16((uint32_t)arg);
    mx = __uint_as_float(pm.a);
    arg = (int)pa.a;
    pick_max(mx, arg, __uint_as_float(pm.b), (int)pa.b);
    pm = swap32(__float_as_uint(mx));
    pa = swap32((uint32_t)arg);
    mx = __uint_as_float(pm.a);
    arg = (int)pa.a;
    pick_max(mx, arg, __uint_as_float(pm.b), (int)pa.b);
}

__device__ inline uint32_t word_of(const uint4& x, int i) {
    return i == 0 ? x.x : i == 1 ? x.y : i == 2 ? x.z : x.w;
}

typedef uint32_t fkv_v2u __attribute__((ext_vector_type(2)));
typedef uint32_t fkv_v4u __attribute__((ext_vector_type(4)));
#define FKV_LDS __attribute__((address_space(3)))
// constant memory: read-only for the duration of a launch (scalar loads)
#define FKV_CONST __attribute__((address_space(4)))

// Workgroup barrier for LDS traffic only: waits for the wave's own LDS
// operations, not for its vector-memory loads (a __syncthreads would also
// drain LDS-DMA transfers still in flight).  One asm block, so no memory
// access moves across it.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 32-bit LDS address of a pointer into a __shared__ array.
__device__ inline uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const FKV_LDS void*)p;
}

// q as the B operand of the score MFMA, in LDS as [qd][s][j][4 halves].
template <int NS>
struct QOperand {
    const uint16_t* qs;
    int base;  // j * 4 for lane quad position j
    __device__ QOperand fresh() const {
        QOperand r = *this;
        asm volatile("" : "+v"(r.base));
        return r;
    }
    __device__ fkv_h4 operator()(int qd, int s) const {
        uint2 v;
        __builtin_memcpy(&v, qs + base + (qd * NS + s) * 16, 8);
        return __builtin_bit_cast(fkv_h4, v);
    }
    // Operands of k-steps s0..s0+7 of quad qd, read by one asm block that
    // waits for its own LDS reads (used where LDS DMA is in flight: the
    // compiler would otherwise drain every DMA before any LDS read).
    __device__ void read8(int qd, int s0, fkv_h4 (&o)[8]) const {
        const uint32_t addr = lds_addr(qs + base + (qd * NS + s0) * 16);
        fkv_v2u r0, r1, r2, r3, r4, r5, r6, r7;
        asm volatile(
            "ds_read_b64 %0, %8\n"
            "ds_read_b64 %1, %8 offset:32\n"
            "ds_read_b64 %2, %8 offset:64\n"
            "ds_read_b64 %3, %8 offset:96\n"
            "ds_read_b64 %4, %8 offset:128\n"
            "ds_read_b64 %5, %8 offset:160\n"
            "ds_read_b64 %6, %8 offset:192\n"
            "ds_read_b64 %7, %8 offset:224\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&v"(r4), "=&v"(r5), "=&v"(r6), "=&v"(r7)
            : "v"(addr)
            : "memory");
        o[0] = __builtin_bit_cast(fkv_h4, r0);
        o[1] = __builtin_bit_cast(fkv_h4, r1);
        o[2] = __builtin_bit_cast(fkv_h4, r2);
        o[3] = __builtin_bit_cast(fkv_h4, r3);
        o[4] = __builtin_bit_cast(fkv_h4, r4);
        o[5] = __builtin_bit_cast(fkv_h4, r5);
        o[6] = __builtin_bit_cast(fkv_h4, r6);
        o[7] = __builtin_bit_cast(fkv_h4, r7);
    }
    // read8x2 over 16 k-steps: one wait for 32 reads
    __device__ void read16x2(int s0, fkv_h4 (&o)[2][16]) const {
        static_assert(NS * 32 + 480 < 65536, "ds_read offset");
        const uint32_t addr = lds_addr(qs + base + s0 * 16);
        fkv_v2u r[32];
        asm volatile(
            "ds_read_b64 %0, %32\n"
            "ds_read_b64 %1, %32 offset:32\n"
            "ds_read_b64 %2, %32 offset:64\n"
            "ds_read_b64 %3, %32 offset:96\n"
            "ds_read_b64 %4, %32 offset:128\n"
            "ds_read_b64 %5, %32 offset:160\n"
            "ds_read_b64 %6, %32 offset:192\n"
            "ds_read_b64 %7, %32 offset:224\n"
            "ds_read_b64 %8, %32 offset:256\n"
            "ds_read_b64 %9, %32 offset:288\n"
            "ds_read_b64 %10, %32 offset:320\n"
            "ds_read_b64 %11, %32 offset:352\n"
            "ds_read_b64 %12, %32 offset:384\n"
            "ds_read_b64 %13, %32 offset:416\n"
            "ds_read_b64 %14, %32 offset:448\n"
            "ds_read_b64 %15, %32 offset:480\n"
            "ds_read_b64 %16, %32 offset:%33\n"
            "ds_read_b64 %17, %32 offset:%33+32\n"
            "ds_read_b64 %18, %32 offset:%33+64\n"
            "ds_read_b64 %19, %32 offset:%33+96\n"
            "ds_read_b64 %20, %32 offset:%33+128\n"
            "ds_read_b64 %21, %32 offset:%33+160\n"
            "ds_read_b64 %22, %32 offset:%33+192\n"
            "ds_read_b64 %23, %32 offset:%33+224\n"
            "ds_read_b64 %24, %32 offset:%33+256\n"
            "ds_read_b64 %25, %32 offset:%33+288\n"
            "ds_read_b64 %26, %32 offset:%33+320\n"
            "ds_read_b64 %27, %32 offset:%33+352\n"
            "ds_read_b64 %28, %32 offset:%33+384\n"
            "ds_read_b64 %29, %32 offset:%33+416\n"
            "ds_read_b64 %30, %32 offset:%33+448\n"
            "ds_read_b64 %31, %32 offset:%33+480\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7]), "=&v"(r[8]), "=&v"(r[9]), "=&v"(r[10]), "=&v"(r[11]), "=&v"(r[12]), "=&v"(r[13]), "=&v"(r[14]), "=&v"(r[15]), "=&v"(r[16]), "=&v"(r[17]), "=&v"(r[18]), "=&v"(r[19]), "=&v"(r[20]), "=&v"(r[21]), "=&v"(r[22]), "=&v"(r[23]), "=&v"(r[24]), "=&v"(r[25]), "=&v"(r[26]), "=&v"(r[27]), "=&v"(r[28]), "=&v"(r[29]), "=&v"(r[30]), "=&v"(r[31])
            : "v"(addr), "n"(NS * 32)
            : "memory");
#pragma unroll
        for (int i = 0; i < 16; i++) {
            o[0][i] = __builtin_bit_cast(fkv_h4, r[i]);
            o[1][i] = __builtin_bit_cast(fkv_h4, r[16 + i]);
        }
    }
    // read8 of quads 0 and 1 in one asm block: one wait for both
    __device__ void read8x2(int s0, fkv_h4 (&o)[2][8]) const {
        static_assert(NS * 32 + 224 < 65536, "ds_read offset");
        const uint32_t addr = lds_addr(qs + base + s0 * 16);
        fkv_v2u r[16];
        asm volatile(
            "ds_read_b64 %0, %16\n"
            "ds_read_b64 %1, %16 offset:32\n"
            "ds_read_b64 %2, %16 offset:64\n"
            "ds_read_b64 %3, %16 offset:96\n"
            "ds_read_b64 %4, %16 offset:128\n"
            "ds_read_b64 %5, %16 offset:160\n"
            "ds_read_b64 %6, %16 offset:192\n"
            "ds_read_b64 %7, %16 offset:224\n"
            "ds_read_b64 %8, %16 offset:%17\n"
            "ds_read_b64 %9, %16 offset:%17+32\n"
            "ds_read_b64 %10, %16 offset:%17+64\n"
            "ds_read_b64 %11, %16 offset:%17+96\n"
            "ds_read_b64 %12, %16 offset:%17+128\n"
            "ds_read_b64 %13, %16 offset:%17+160\n"
            "ds_read_b64 %14, %16 offset:%17+192\n"
            "ds_read_b64 %15, %16 offset:%17+224\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]),
              "=&v"(r[7]), "=&v"(r[8]), "=&v"(r[9]), "=&v"(r[10]), "=&v"(r[11]), "=&v"(r[12]), "=&v"(r[13]),
              "=&v"(r[14]), "=&v"(r[15])
            : "v"(addr), "n"(NS * 32)
            : "memory");
#pragma unroll
        for (int i = 0; i < 8; i++) {
            o[0][i] = __builtin_bit_cast(fkv_h4, r[i]);
            o[1][i] = __builtin_bit_cast(fkv_h4, r[8 + i]);
        }
    }
    // N (2, 4 or 8) k-steps s0.. of quad qd (see lds_q)
    template <int N>
    __device__ void readn(int qd, int s0, fkv_h4 (&o)[N]) const;
};

// q as the B operand of the score MFMA held in registers for the whole
// launch (rows of one head quad): read once from the LDS operand array after
// the prologue, so tiles issue no LDS reads (and no waits) for the query.
template <int NS>
struct QReg {
    fkv_h4 q[NS];
    __device__ void load(const QOperand<NS>& src) {
#pragma unroll
        for (int s0 = 0; s0 < NS; s0 += 8) {
            fkv_h4 t[8];
            src.read8(0, s0, t);
#pragma unroll
            for (int i = 0; i < 8; i++) q[s0 + i] = t[i];
        }
    }
    __device__ QReg fresh() const { return *this; }
    __device__ fkv_h4 operator()(int, int s) const { return q[s]; }
    __device__ void read8(int, int s0, fkv_h4 (&o)[8]) const {
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = q[s0 + i];
    }
    template <int N>
    __device__ void readn(int, int s0, fkv_h4 (&o)[N]) const {
#pragma unroll
        for (int i = 0; i < N; i++) o[i] = q[s0 + i];
    }
};

template <int D, int NQ>
struct Lane {
    // per head quad: this lane tracks head 4*qd + (lane % 4)
    float m[NQ], lsum[NQ], mn[NQ], mx[NQ];
    // INT4 correction terms, sum of p*(zero + 7.5*scale) - 23.5*w over the
    // lane's tokens (w: the fp16 P.V weight; removes the +16 decode offset
    // and the 7.5 centring).  Per token V: index 0; group-32 V: [dh] for the
    // group of the lane's own half, [D/64 + dh] for the other half's group.
    float zsum[NQ][D / 32];
    int arg[NQ];
    fkv_f4 acc[NQ][D / 64];  // acc[qd][dh][i] = O[head 4qd+i][dim 64dh + lane]
};

// Rescale head quad qd's running state by alpha (the lane's head's factor;
// the accumulators of head i of the quad take lane i's factor).
template <int D, int NQ>
__device__ inline void rescale(Lane<D, NQ>& st, int qd, float alpha) {
    st.lsum[qd] *= alpha;
#pragma unroll
    for (int z = 0; z < D / 32; z++) {
        st.zsum[qd][z] *= alpha;
    }
    const float a0 = quad_bcast<0>(alpha), a1 = quad_bcast<1>(alpha);
    const float a2 = quad_bcast<2>(alpha), a3 = quad_bcast<3>(alpha);
#pragma unroll
    for (int dh = 0; dh < D / 64; dh++) {
        st.acc[qd][dh][0] *= a0;
        st.acc[qd][dh][1] *= a1;
        st.acc[qd][dh][2] *= a2;
        st.acc[qd][dh][3] *= a3;
    }
}

// One 64-token far tile as loaded from the blob: E4M3 keys (lane = token,
// 16 codes per chunk), INT4 values (lane = dim), per-token scale|zero of the
// lane's 4-token group.
template <int D>
struct FarTile {
    uint4 k[D / 16];
    uint4 v[D / 32];
    uint4 sz;
};

// Far tile record -> an LDS slot with gfx950's direct global->LDS loads
// (global_load_lds_dwordx4, non-temporal): the K|V sections as 1-KB chunks
// by the whole wave, then the 256-byte SZ section by lanes 0..15.  Issues
// far_dma_ops<D>() vector-memory instructions; completion is tracked with
// vmcnt by the caller (the compiler does not order LDS reads after them).
template <int D>
constexpr int far_dma_ops() { return 3 * D / 32 + 1; }

template <int D>
__device__ inline void dma_far(const AttnArgs& a, int64_t bkv, int tile, int lane, uint8_t* slot) {
    const uint8_t* rec = a.blob + a.L.far + far_rec_index(a.L, bkv, tile) * (int64_t)a.L.far_rec;
#pragma unroll
    for (int c = 0; c < 3 * D / 32; c++)
        __builtin_amdgcn_global_load_lds((const void*)(rec + c * 1024 + lane * 16), (FKV_LDS void*)(slot + c * 1024), 16,
                                         0, 2);
    // the 256-byte SZ section by lanes 0..15 (a single lane-conditional
    // instruction: the branch cannot be merged with another one, see dma_tq)
    if (lane < 16)
        __builtin_amdgcn_global_load_lds((const void*)(rec + far_sz_section(D) + lane * 16),
                                         (FKV_LDS void*)(slot + far_sz_section(D)), 16, 0, 2);
}

__device__ inline uint4 u4_of(fkv_v4u v) { return make_uint4(v.x, v.y, v.z, v.w); }

// Part `part` of NP of one half (K: 0 or V: 1) of a near-tier tile -> an
// LDS slot: D / (8 NP) 1-KB chunks (the tile layout is already
// chunk-major: K chunk c = dims 8c..8c+7, V chunks of dim half dh are
// 8dh..8dh+7).
template <int D, int NP = 1>
__device__ inline void dma_near(const AttnArgs& a, int64_t bkv, int tile, int half, int part, int lane,
                                uint8_t* slot) {
    constexpr int NC = D / 8 / NP;
    const uint8_t* src = a.blob + (half ? a.L.near_v : a.L.near_k) +
                         (bkv * a.L.Na_pad + (int64_t)tile * kTile) * D * 2 + part * NC * 1024;
#pragma unroll
    for (int c = 0; c < NC; c++)
        __builtin_amdgcn_global_load_lds((const void*)(src + c * 1024 + lane * 16), (FKV_LDS void*)(slot + c * 1024), 16,
                                         0, 2);
}

// The lane's operands of a far tile held in an LDS slot, read by one asm
// block that waits for its own LDS reads (see QOperand::read8).
__device__ inline void lds_far(FarTile<128>& r, const uint8_t* slot, int lane) {
    const uint32_t a = lds_addr(slot + lane * 16), z = lds_addr(slot + far_sz_section(128) + (lane >> 2) * 16);
    fkv_v4u c0, c1, c2, c3, c4, c5, c6, c7, c8, c9, c10, c11, sz;
    asm volatile(
        "ds_read_b128 %0, %13\n"
        "ds_read_b128 %1, %13 offset:1024\n"
        "ds_read_b128 %2, %13 offset:2048\n"
        "ds_read_b128 %3, %13 offset:3072\n"
        "ds_read_b128 %4, %13 offset:4096\n"
        "ds_read_b128 %5, %13 offset:5120\n"
        "ds_read_b128 %6, %13 offset:6144\n"
        "ds_read_b128 %7, %13 offset:7168\n"
        "ds_read_b128 %8, %13 offset:8192\n"
        "ds_read_b128 %9, %13 offset:9216\n"
        "ds_read_b128 %10, %13 offset:10240\n"
        "ds_read_b128 %11, %13 offset:11264\n"
        "ds_read_b128 %12, %14\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(c0), "=&v"(c1), "=&v"(c2), "=&v"(c3), "=&v"(c4), "=&v"(c5), "=&v"(c6), "=&v"(c7), "=&v"(c8),
          "=&v"(c9), "=&v"(c10), "=&v"(c11), "=&v"(sz)
        : "v"(a), "v"(z)
        : "memory");
    r.k[0] = u4_of(c0); r.k[1] = u4_of(c1); r.k[2] = u4_of(c2); r.k[3] = u4_of(c3);
    r.k[4] = u4_of(c4); r.k[5] = u4_of(c5); r.k[6] = u4_of(c6); r.k[7] = u4_of(c7);
    r.v[0] = u4_of(c8); r.v[1] = u4_of(c9); r.v[2] = u4_of(c10); r.v[3] = u4_of(c11);
    r.sz = u4_of(sz);
}

__device__ inline void lds_far(FarTile<64>& r, const uint8_t* slot, int lane) {
    const uint32_t a = lds_addr(slot + lane * 16), z = lds_addr(slot + far_sz_section(64) + (lane >> 2) * 16);
    fkv_v4u c0, c1, c2, c3, c4, c5, sz;
    asm volatile(
        "ds_read_b128 %0, %7\n"
        "ds_read_b128 %1, %7 offset:1024\n"
        "ds_read_b128 %2, %7 offset:2048\n"
        "ds_read_b128 %3, %7 offset:3072\n"
        "ds_read_b128 %4, %7 offset:4096\n"
        "ds_read_b128 %5, %7 offset:5120\n"
        "ds_read_b128 %6, %8\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(c0), "=&v"(c1), "=&v"(c2), "=&v"(c3), "=&v"(c4), "=&v"(c5), "=&v"(sz)
        : "v"(a), "v"(z)
        : "memory");
    r.k[0] = u4_of(c0); r.k[1] = u4_of(c1); r.k[2] = u4_of(c2); r.k[3] = u4_of(c3);
    r.v[0] = u4_of(c4); r.v[1] = u4_of(c5);
    r.sz = u4_of(sz);
}

// out = acc / l (fp16), spike flag and token for ng heads of one record set
template <int D, bool EXT = false>
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
        if (EXT && a.thr) a.thr[o] = mn + a.spike_margin;
    }
}

// P.V step of 4-token group G: the weights of the group (block G of each
// quad's w4) broadcast to all 16 blocks, times the group's values of dims
// 64dh + 4b..4b+3; one value operand serves every head quad.
template <int D, int NQ, int G, typename VOp>
__device__ inline void pv_group(Lane<D, NQ>& st, const fkv_h4 (&w4)[NQ], VOp vop) {
#pragma unroll
    for (int dh = 0; dh < D / 64; dh++) {
        const fkv_h4 v = vop(G, dh);
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) st.acc[qd][dh] = mfma4<G>(w4[qd], v, st.acc[qd][dh]);
    }
}

// The MFMAs of group G with its value operands already formed.
template <int D, int NQ, int G>
__device__ inline void pv_mfma(Lane<D, NQ>& st, const fkv_h4 (&w4)[NQ], const fkv_h4 (&v)[D / 64]) {
#pragma unroll
    for (int dh = 0; dh < D / 64; dh++)
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) st.acc[qd][dh] = mfma4<G>(w4[qd], v[dh], st.acc[qd][dh]);
}

// Groups G0 .. G0 + 7: every value operand formed (or loaded) before the
// first MFMA: an operand feeding the next MFMA directly costs wait states,
// and operands gathered from global memory then share one round trip.
template <int D, int NQ, int G0, typename VOp>
__device__ inline void pv_batch8(Lane<D, NQ>& st, const fkv_h4 (&w4)[NQ], VOp vop) {
    fkv_h4 v[8][D / 64];
#pragma unroll
    for (int g = 0; g < 8; g++)
#pragma unroll
        for (int dh = 0; dh < D / 64; dh++) v[g][dh] = vop(G0 + g, dh);
    pv_mfma<D, NQ, G0 + 0>(st, w4, v[0]);
    pv_mfma<D, NQ, G0 + 1>(st, w4, v[1]);
    pv_mfma<D, NQ, G0 + 2>(st, w4, v[2]);
    pv_mfma<D, NQ, G0 + 3>(st, w4, v[3]);
    pv_mfma<D, NQ, G0 + 4>(st, w4, v[4]);
    pv_mfma<D, NQ, G0 + 5>(st, w4, v[5]);
    pv_mfma<D, NQ, G0 + 6>(st, w4, v[6]);
    pv_mfma<D, NQ, G0 + 7>(st, w4, v[7]);
}

// Groups G0 .. G0 + GB - 1 (GB = 4 or 8) of a tile whose values are INT4
// dword pairs: pop(j, dh) is the pair of 4-token groups 4j .. 4j + 3 of
// 64-dim half dh; every operand of the batch is formed before its first
// MFMA.
template <int D, int NQ, int G0, int GB, typename PairOp>
__device__ inline void pv_pair_batch(Lane<D, NQ>& st, const fkv_h4 (&w4)[NQ], PairOp pop) {
    fkv_h4 v[GB][D / 64];
#pragma unroll
    for (int dh = 0; dh < D / 64; dh++)
#pragma unroll
        for (int j = 0; j < GB / 4; j++) {
            fkv_h4 o[4];
            int4x4_pair(pop(G0 / 4 + j, dh), o);
#pragma unroll
            for (int i = 0; i < 4; i++) v[4 * j + i][dh] = o[i];
        }
    pv_mfma<D, NQ, G0 + 0>(st, w4, v[0]);
    pv_mfma<D, NQ, G0 + 1>(st, w4, v[1]);
    pv_mfma<D, NQ, G0 + 2>(st, w4, v[2]);
    pv_mfma<D, NQ, G0 + 3>(st, w4, v[3]);
    if constexpr (GB == 8) {
        pv_mfma<D, NQ, G0 + 4>(st, w4, v[4]);
        pv_mfma<D, NQ, G0 + 5>(st, w4, v[5]);
        pv_mfma<D, NQ, G0 + 6>(st, w4, v[6]);
        pv_mfma<D, NQ, G0 + 7>(st, w4, v[7]);
    }
}

// The P.V of one 64-token tile from INT4 dword pairs, GB groups per batch.
template <int D, int NQ, int GB, typename PairOp>
__device__ inline void pv_pairs(Lane<D, NQ>& st, const fkv_h4 (&w4)[NQ], PairOp pop) {
    static_assert(GB == 4 || GB == 8, "batches of 4 or 8 groups");
    if constexpr (GB == 8) {
        pv_pair_batch<D, NQ, 0, 8>(st, w4, pop);
        pv_pair_batch<D, NQ, 8, 8>(st, w4, pop);
    } else {
        pv_pair_batch<D, NQ, 0, 4>(st, w4, pop);
        pv_pair_batch<D, NQ, 4, 4>(st, w4, pop);
        pv_pair_batch<D, NQ, 8, 4>(st, w4, pop);
        pv_pair_batch<D, NQ, 12, 4>(st, w4, pop);
    }
}

// The P.V of one 64-token tile over the 16 groups of 4 tokens, the value
// operands formed BATCH groups at a time (1 or 8).
template <int D, int NQ, int BATCH = 1, typename VOp>
__device__ inline void pv_all(Lane<D, NQ>& st, const fkv_h4 (&w4)[NQ], VOp vop) {
    static_assert(BATCH == 1 || BATCH == 8, "batch of 1 or 8 groups");
    if constexpr (BATCH == 8) {
        pv_batch8<D, NQ, 0>(st, w4, vop);
        pv_batch8<D, NQ, 8>(st, w4, vop);
    } else {
        pv_group<D, NQ, 0>(st, w4, vop);
        pv_group<D, NQ, 1>(st, w4, vop);
        pv_group<D, NQ, 2>(st, w4, vop);
        pv_group<D, NQ, 3>(st, w4, vop);
        pv_group<D, NQ, 4>(st, w4, vop);
        pv_group<D, NQ, 5>(st, w4, vop);
        pv_group<D, NQ, 6>(st, w4, vop);
        pv_group<D, NQ, 7>(st, w4, vop);
        pv_group<D, NQ, 8>(st, w4, vop);
        pv_group<D, NQ, 9>(st, w4, vop);
        pv_group<D, NQ, 10>(st, w4, vop);
        pv_group<D, NQ, 11>(st, w4, vop);
        pv_group<D, NQ, 12>(st, w4, vop);
        pv_group<D, NQ, 13>(st, w4, vop);
        pv_group<D, NQ, 14>(st, w4, vop);
        pv_group<D, NQ, 15>(st, w4, vop);
    }
}

// Online-softmax update of head quad qd for one 64-token tile (scores s[e]
// of tokens 4*(lane/4) + e, head 4qd + lane%4).  Writes the fp16 P.V
// weights of the lane (far tiles: p * per-token scale; the zero point and
// the INT4 decode offset go to per-head scalars) and returns whether any
// weight of the lane is non-zero.
template <int D, int NQ, bool FAR>
__device__ inline bool softmax_w(Lane<D, NQ>& st, int qd, const float (&s)[4], const uint32_t (&sz)[4],
                                 fkv_h4& w4, float* tile_max = nullptr) {
    float cmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    cmax = head_max(cmax);
    if (tile_max) *tile_max = cmax;
    const float m_new = fmaxf(st.m[qd], cmax);
    if (__builtin_amdgcn_ballot_w64(m_new > st.m[qd])) {
        rescale<D, NQ>(st, qd, m_new > st.m[qd] ? __expf(st.m[qd] - m_new) : 1.0f);
        st.m[qd] = m_new;
    }
    _Float16 wh[4];
    float pe[4], ce[4];
    bool any = false;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float p = 0.f;
        if (FAR) {
            if (s[e] >= st.m[qd] - 16.0f) p = __expf(s[e] - st.m[qd]);  // score-gated V
        } else if (s[e] != -INFINITY) {
            p = __expf(s[e] - st.m[qd]);
        }
        pe[e] = p;
        if (FAR) {
            const float vs = h2f((uint16_t)(sz[e] & 0xFFFF));
            const float vz = h2f((uint16_t)(sz[e] >> 16));
            wh[e] = (_Float16)(p * vs);
            // value = vs*(c - 7.5) + (vz + 7.5*vs) and the MFMA sees wh*(16 + c):
            // the token adds p*(vz + 7.5*vs) - 23.5*wh
            ce[e] = fmaf(-23.5f, (float)wh[e], p * (vz + 7.5f * vs));
        } else {
            wh[e] = (_Float16)p;
        }
        any |= p > 0.f;
    }
    st.lsum[qd] += (pe[0] + pe[1]) + (pe[2] + pe[3]);
    if (FAR) st.zsum[qd][0] += (ce[0] + ce[1]) + (ce[2] + ce[3]);
    w4 = fkv_h4{wh[0], wh[1], wh[2], wh[3]};
    return any;
}

// Where a wave stores its far tiles' per-head maxima for the top-K spike
// selection: p = the row's first head's tile maxima (NULL: spike_k = 1, no
// stores), stride = far tiles per head, ng = heads of the row.
struct SpikeTiles {
    float* p;
    int stride, ng;
};

// The far tile's maximum score of each head of quad qd (c: the softmax's
// tile maximum, lane % 4 = head of the quad, -inf past the far tier),
// stored by lanes 0-3.  Only the top-K kernels (SPK) store.
template <bool SPK>
__device__ inline void store_tile_max(const SpikeTiles& sp, int qd, int tile, float c) {
    if (!SPK) return;
    const int lane = (int)threadIdx.x % kWave, h = 4 * qd + lane;
    if (lane < 4 && h < sp.ng) sp.p[(int64_t)h * sp.stride + tile] = c;
}

// Scores, spike tracking, softmax and P.V of one loaded far tile.
template <int D, int NQ, bool SPK, typename QOp>
__device__ inline void far_compute(Lane<D, NQ>& st, const FarTile<D>& r, int tile, int F, int blk,
                                   float inv_sqrt_d, const QOp& q_lds, const SpikeTiles& sp) {
    constexpr int NS = D / 4;
    const uint32_t sz[4] = {r.sz.x, r.sz.y, r.sz.z, r.sz.w};
    fkv_f4 sacc[NQ];
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) sacc[qd] = fkv_f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (NQ == 2) {
        // two quads: 16 k-steps of both quads' operands per LDS batch
#pragma unroll
        for (int s0 = 0; s0 < NS; s0 += 16) {
            fkv_h4 q16[2][16];
            q_lds.read16x2(s0, q16);
            // every key operand of the batch converted before the first MFMA
            // (a conversion feeding the next MFMA directly costs wait states)
            fkv_h4 k16[16];
#pragma unroll
            for (int s = s0; s < s0 + 16; s++) k16[s - s0] = e4m3x4(word_of(r.k[s >> 2], s & 3));
#pragma unroll
            for (int s = s0; s < s0 + 16; s++) {
                sacc[0] = mfma4_local(k16[s - s0], q16[0][s - s0], sacc[0]);
                sacc[1] = mfma4_local(k16[s - s0], q16[1][s - s0], sacc[1]);
            }
        }
    } else {
#pragma unroll
        for (int s0 = 0; s0 < NS; s0 += 8) {
            fkv_h4 q8[NQ][8];
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) q_lds.read8(qd, s0, q8[qd]);
            fkv_h4 k8[8];
#pragma unroll
            for (int s = s0; s < s0 + 8; s++) k8[s - s0] = e4m3x4(word_of(r.k[s >> 2], s & 3));
#pragma unroll
            for (int s = s0; s < s0 + 8; s++)
#pragma unroll
                for (int qd = 0; qd < NQ; qd++) sacc[qd] = mfma4_local(k8[s - s0], q8[qd][s - s0], sacc[qd]);
        }
    }
    fkv_h4 w4[NQ];
    bool any = false;
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = tile * kTile + 4 * blk + e;
            const float sv = sacc[qd][e] * inv_sqrt_d;
            const bool ok = t < F;
            sc[e] = ok ? sv : -INFINITY;
            if (ok && sv > st.mx[qd]) { st.mx[qd] = sv; st.arg[qd] = t; }  // first index of the max
        }
        float cmax = -INFINITY;  // set by the softmax where SPK
        any |= softmax_w<D, NQ, true>(st, qd, sc, sz, w4[qd], SPK ? &cmax : nullptr);
        store_tile_max<SPK>(sp, qd, tile, cmax);
    }
    if (__builtin_amdgcn_ballot_w64(any) == 0) return;  // whole tile gated away
    // dword u = 8 dh + g / 2 of the section holds group g of half dh.  One
    // head quad: operands in batches of 8 groups, from dword pairs (pair j =
    // dwords 8 dh + 2j, + 1).  More quads: group by group (batches of
    // operands there cost more accumulator moves than the pairs save).
    if constexpr (NQ == 1) {
        pv_pairs<D, NQ, 8>(st, w4, [&](int j, int dh) {
            const uint4& x = r.v[dh * 2 + (j >> 1)];
            return (j & 1) ? ((uint64_t)x.w << 32) | x.z : ((uint64_t)x.y << 32) | x.x;
        });
    } else {
        pv_all<D, NQ, 1>(st, w4, [&](int g, int dh) {
            const int u = dh * 8 + (g >> 1);
            return int4x4(word_of(r.v[u >> 2], u & 3), g & 1);
        });
    }
}

// ---------------------------------------------------------------------------
// TurboQuant far tiles (fmt 1): 2-bit Lloyd-Max keys + 1-bit QJL sketch,
// 2-bit values with one fp16 scale per 32 dims
// (csrc/kernels/foveated_attn.metal:486-767)
// ---------------------------------------------------------------------------
//
// Keys: the centroid of code c is alpha + beta*sh + gamma*sl + delta*sh*sl
// over the two +-1 index bits, so q_rot . cb[idx] is a sum of +-1 dot
// products.  The blob holds the bits as complemented planes in which a
// pair of tokens' bits sits at bits 15-i / 31-i of a dword: shifting by i
// and masking with 0x80008000 | 0x3C003C00 yields the two fp16 +-1
// operands, so each 4-dim k-step is three exact MFMAs (high bit, low bit,
// QJL sign) against the fp16 rotated / sketched query.
// Values: level(c) = lvh*sh + lvl*sl times the group scale, and the
// reference's levels {-1, -0.333333, 0.333333, 1} give lvh = 2*lvl (to 5e-7
// relative, checked when the handle is created): the high-bit plane
// expands to +-2 and the low-bit plane to +-1, and both take the one
// weight p * scale * lvl.  The scale
// differs between the two 32-dim groups of a 64-lane P.V block, so the
// weights carry it: with cbsz = 3 the MFMA broadcasts block a's A operand
// to blocks 0-7 and block 8+a's to blocks 8-15, i.e. lanes 0-31 (group
// 2dh) take tokens 4a.. and lanes 32-63 (group 2dh+1) take tokens 32+4a..
// of the lane's own half; a second pass takes the other half's tokens,
// whose weights come across with v_permlane32_swap.  Every lane's weights
// are therefore scaled by its own group's scale.

template <int D>
constexpr int tq_dma_ops() { return D == 128 ? 6 : 4; }

// TurboQuant record -> LDS slot: the KP | VP sections (40*D bytes) as 1 KB
// chunks (D = 64 ends with half a chunk), then SC | NG in one op.
template <int D>
__device__ inline void dma_tq(const AttnArgs& a, int64_t bkv, int tile, int lane, uint8_t* slot) {
    const uint8_t* rec = a.blob + a.L.far + far_rec_index(a.L, bkv, tile) * (int64_t)a.L.far_rec;
    constexpr int KPV = 40 * D, TAIL = 4 * D + 256;
#pragma unroll
    for (int c = 0; c < KPV / 1024; c++)
        __builtin_amdgcn_global_load_lds((const void*)(rec + c * 1024 + lane * 16), (FKV_LDS void*)(slot + c * 1024), 16,
                                         0, 2);
    // Whole-wave instructions: the LDS address operand (M0) must be
    // wave-uniform, and lane-divergent branches around consecutive LDS-DMA
    // builtins can be tail-merged by the compiler into one instruction whose
    // M0 comes from the first active lane.  The partial chunk's upper lanes
    // read the first TAIL bytes, which the next instruction writes to the
    // same LDS bytes; the TAIL's upper lanes repeat lower addresses (same
    // cache lines) and land past the record in the slot.
    if constexpr (KPV % 1024 != 0)
        __builtin_amdgcn_global_load_lds((const void*)(rec + (KPV / 1024) * 1024 + lane * 16),
                                         (FKV_LDS void*)(slot + (KPV / 1024) * 1024), 16, 0, 2);
    constexpr int TL = TAIL / 16;  // lanes of the tail
    __builtin_amdgcn_global_load_lds((const void*)(rec + KPV + (lane < TL ? lane : lane - (64 - TL)) * 16),
                                     (FKV_LDS void*)(slot + KPV), 16, 0, 2);
}

// The lane's operands of a TurboQuant tile.
template <int D>
struct TqTile {
    fkv_v4u kp[3];  // key planes of the lane's token (D = 64: .x/.y only)
    fkv_v4u v[D / 64];   // value planes of dim 64dh + lane: hi own, hi other, lo own, lo other
    fkv_v4u so;  // scales of the lane's 4 tokens in the lane's groups 2dh + half, [e][dh] fp16 (D = 64: .x/.y)
    fkv_v4u sx;  // ... of the other half's 4 tokens (block blk ^ 8)
    fkv_v4u ng;  // norm | gamma << 16 of the lane's 4 tokens
};

__device__ inline void lds_tq(TqTile<128>& r, const uint8_t* slot, int lane) {
    const int blk = lane >> 2, half = lane >> 5;
    const uint32_t a = lds_addr(slot + lane * 16);
    const uint32_t so = lds_addr(slot + tq_sc_section(128) + tq_sc_index(128, blk, half, 0, 0) * 2);
    const uint32_t sx = lds_addr(slot + tq_sc_section(128) + tq_sc_index(128, blk ^ 8, half, 0, 0) * 2);
    const uint32_t ng = lds_addr(slot + tq_ng_section(128) + blk * 16);
    asm volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %8 offset:1024\n"
        "ds_read_b128 %2, %8 offset:2048\n"
        "ds_read_b128 %3, %8 offset:3072\n"
        "ds_read_b128 %4, %8 offset:4096\n"
        "ds_read_b128 %5, %9\n"
        "ds_read_b128 %6, %10\n"
        "ds_read_b128 %7, %11\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r.kp[0]), "=&v"(r.kp[1]), "=&v"(r.kp[2]), "=&v"(r.v[0]), "=&v"(r.v[1]), "=&v"(r.so), "=&v"(r.sx),
          "=&v"(r.ng)
        : "v"(a), "v"(so), "v"(sx), "v"(ng)
        : "memory");
}

__device__ inline void lds_tq(TqTile<64>& r, const uint8_t* slot, int lane) {
    const int blk = lane >> 2, half = lane >> 5;
    const uint32_t a = lds_addr(slot + lane * 8);
    const uint32_t v = lds_addr(slot + tq_vp_section(64) + lane * 16);
    const uint32_t so = lds_addr(slot + tq_sc_section(64) + tq_sc_index(64, blk, half, 0, 0) * 2);
    const uint32_t sx = lds_addr(slot + tq_sc_section(64) + tq_sc_index(64, blk ^ 8, half, 0, 0) * 2);
    const uint32_t ng = lds_addr(slot + tq_ng_section(64) + blk * 16);
    fkv_v2u k0, k1, k2, s0, s1;
    asm volatile(
        "ds_read_b64 %0, %7\n"
        "ds_read_b64 %1, %7 offset:512\n"
        "ds_read_b64 %2, %7 offset:1024\n"
        "ds_read_b128 %3, %8\n"
        "ds_read_b64 %4, %9\n"
        "ds_read_b64 %5, %10\n"
        "ds_read_b128 %6, %11\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k0), "=&v"(k1), "=&v"(k2), "=&v"(r.v[0]), "=&v"(s0), "=&v"(s1), "=&v"(r.ng)
        : "v"(a), "v"(v), "v"(so), "v"(sx), "v"(ng)
        : "memory");
    r.kp[0] = fkv_v4u{k0.x, k0.y, 0u, 0u};
    r.kp[1] = fkv_v4u{k1.x, k1.y, 0u, 0u};
    r.kp[2] = fkv_v4u{k2.x, k2.y, 0u, 0u};
    r.so = fkv_v4u{s0.x, s0.y, 0u, 0u};
    r.sx = fkv_v4u{s1.x, s1.y, 0u, 0u};
}

// Bit-select constants held in registers: with the mask and the fp16 +1
// pair opaque to constant folding the compiler selects one v_bfi_b32 per
// word (gfx9 VOP3 takes no literals, so folded constants cost an AND and
// an OR).  The empty asm emits no instruction.
struct PmConst {
    uint32_t m, c, c2;  // sign mask, fp16 pairs (1, 1) and (2, 2)
    __device__ static PmConst make() {
        PmConst k{0x80008000u, 0x3C003C00u, 0x40004000u};
        asm volatile("" : "+s"(k.m));
        asm volatile("" : "+v"(k.c));
        asm volatile("" : "+v"(k.c2));
        return k;
    }
};

// two fp16 values +-c from the bits at 15 and 31 (set = negative)
__device__ inline uint32_t pm1(uint32_t w, uint32_t m, uint32_t c) { return (w & m) | (c & ~m); }
__device__ inline uint32_t pm1(uint32_t w, const PmConst& k) { return pm1(w, k.m, k.c); }

// A plane word held as the pair (w, w << 1) (high, low dword): one 64-bit
// shift by an even i <= 14 gives w << i and w << (i + 1) together.  The
// high dword also takes the top i bits of w << 1, but they land below bit
// i, never at the bits 15 and 31 that pm1 reads.  The shift amount is made
// opaque (an empty asm on a scalar register), so the compiler keeps the one
// v_lshlrev_b64 instead of splitting a constant shift into two 32-bit
// ones; v_lshlrev_b64 issues at the rate of v_lshlrev_b32.
__device__ inline uint64_t plane_pair(uint32_t w) { return ((uint64_t)w << 32) | (uint64_t)(w << 1); }

// the +-c operand of 4 consecutive dims / tokens (c = 1: k.c, 2: k.c2):
// pairs i, i+1 of the plane word of w2 = plane_pair(w)
__device__ inline fkv_h4 pm1x4(uint64_t w2, int i, const PmConst& k, bool two = false) {
    uint64_t s = w2;
    if (i != 0) {
        uint32_t n = (uint32_t)i;
        asm("" : "+s"(n));
        s = w2 << n;
    }
    const uint32_t c = two ? k.c2 : k.c;
    return h4_of(pm1((uint32_t)(s >> 32), k.m, c), pm1((uint32_t)s, k.m, c));
}

// N q-operand k-steps s0.. of quad qd from an LDS operand array, one asm
// block that waits for its own reads (see QOperand::read8).
template <int N>
__device__ inline void lds_q(const uint16_t* p, fkv_h4 (&o)[N]);
template <>
__device__ inline void lds_q<8>(const uint16_t* p, fkv_h4 (&o)[8]) {
    const uint32_t addr = lds_addr(p);
    fkv_v2u r0, r1, r2, r3, r4, r5, r6, r7;
    asm volatile(
        "ds_read_b64 %0, %8\n"
        "ds_read_b64 %1, %8 offset:32\n"
        "ds_read_b64 %2, %8 offset:64\n"
        "ds_read_b64 %3, %8 offset:96\n"
        "ds_read_b64 %4, %8 offset:128\n"
        "ds_read_b64 %5, %8 offset:160\n"
        "ds_read_b64 %6, %8 offset:192\n"
        "ds_read_b64 %7, %8 offset:224\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&v"(r4), "=&v"(r5), "=&v"(r6), "=&v"(r7)
        : "v"(addr)
        : "memory");
    o[0] = __builtin_bit_cast(fkv_h4, r0); o[1] = __builtin_bit_cast(fkv_h4, r1);
    o[2] = __builtin_bit_cast(fkv_h4, r2); o[3] = __builtin_bit_cast(fkv_h4, r3);
    o[4] = __builtin_bit_cast(fkv_h4, r4); o[5] = __builtin_bit_cast(fkv_h4, r5);
    o[6] = __builtin_bit_cast(fkv_h4, r6); o[7] = __builtin_bit_cast(fkv_h4, r7);
}
template <>
__device__ inline void lds_q<4>(const uint16_t* p, fkv_h4 (&o)[4]) {
    const uint32_t addr = lds_addr(p);
    fkv_v2u r0, r1, r2, r3;
    asm volatile(
        "ds_read_b64 %0, %4\n"
        "ds_read_b64 %1, %4 offset:32\n"
        "ds_read_b64 %2, %4 offset:64\n"
        "ds_read_b64 %3, %4 offset:96\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
        : "v"(addr)
        : "memory");
    o[0] = __builtin_bit_cast(fkv_h4, r0); o[1] = __builtin_bit_cast(fkv_h4, r1);
    o[2] = __builtin_bit_cast(fkv_h4, r2); o[3] = __builtin_bit_cast(fkv_h4, r3);
}
template <>
__device__ inline void lds_q<2>(const uint16_t* p, fkv_h4 (&o)[2]) {
    const uint32_t addr = lds_addr(p);
    fkv_v2u r0, r1;
    asm volatile(
        "ds_read_b64 %0, %2\n"
        "ds_read_b64 %1, %2 offset:32\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r0), "=&v"(r1)
        : "v"(addr)
        : "memory");
    o[0] = __builtin_bit_cast(fkv_h4, r0); o[1] = __builtin_bit_cast(fkv_h4, r1);
}

template <int NS>
template <int N>
__device__ inline void QOperand<NS>::readn(int qd, int s0, fkv_h4 (&o)[N]) const {
    lds_q<N>(qs + base + (qd * NS + s0) * 16, o);
}

// Online-softmax update of head quad qd for a far tile: rescale on a new
// maximum, then the gated weights p (the reference skips V of far tokens
// with s < m - 16, foveated_attn.metal:713).  Returns whether any p > 0.
template <int D, int NQ>
__device__ inline bool tq_softmax(Lane<D, NQ>& st, int qd, const float (&s)[4], float (&p)[4],
                                  float* tile_max = nullptr) {
    float cmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    cmax = head_max(cmax);
    if (tile_max) *tile_max = cmax;
    const float m_new = fmaxf(st.m[qd], cmax);
    if (__builtin_amdgcn_ballot_w64(m_new > st.m[qd])) {
        rescale<D, NQ>(st, qd, m_new > st.m[qd] ? __expf(st.m[qd] - m_new) : 1.0f);
        st.m[qd] = m_new;
    }
    bool any = false;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        p[e] = s[e] >= st.m[qd] - 16.0f ? __expf(s[e] - st.m[qd]) : 0.f;
        st.lsum[qd] += p[e];
        any |= p[e] > 0.f;
    }
    return any;
}

// v_mfma_f32_4x4x4f16 with cbsz = 3: blocks 0-7 take block A's operand,
// blocks 8-15 take block 8+A's.
template <int A>
__device__ inline fkv_f4 mfma4_half(fkv_h4 a, fkv_h4 b, fkv_f4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 3, A, 0);
}

// Step A of the P.V of one tile: 4 MFMAs per head quad into two partial
// sums (own-half and other-half tokens) so consecutive MFMAs do not wait
// on each other; the high-bit planes expand to +-2, the low-bit ones to
// +-1, against one weight per token.
template <int NQ, int A>
__device__ inline void tq_pv_step(fkv_f4 (&po)[NQ], fkv_f4 (&px)[NQ], const uint64_t (&v)[4], const fkv_h4 (&w)[2][NQ],
                                  const PmConst& k) {
    const fkv_h4 b1h = pm1x4(v[0], 2 * A, k, true), b2h = pm1x4(v[1], 2 * A, k, true);
    const fkv_h4 b1l = pm1x4(v[2], 2 * A, k), b2l = pm1x4(v[3], 2 * A, k);
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        po[qd] = mfma4_half<A>(w[0][qd], b1h, po[qd]);
        px[qd] = mfma4_half<A>(w[1][qd], b2h, px[qd]);
        po[qd] = mfma4_half<A>(w[0][qd], b1l, po[qd]);
        px[qd] = mfma4_half<A>(w[1][qd], b2l, px[qd]);
    }
}

// fp16 number i of the scale words s (compile-time i: a low or high half)
__device__ inline float half_of(const fkv_v4u& s, int i) {
    const uint32_t w = s[i >> 1];
    return h2f((uint16_t)((i & 1) ? (w >> 16) : (w & 0xFFFF)));
}

// The other half's copy of v (lane l gets lane l ^ 32's value).
__device__ inline float swap_halves(float v, int half) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(half ? r[0] : r[1]);
}

// The other half's copies of two values in two v_permlane32_swap (each
// swaps the upper half of its first operand with the lower half of its
// second): (x, y) -> ([x.lo, y.lo], [x.hi, y.hi]) -> ([x.hi, x.lo],
// [y.hi, y.lo]), with no per-lane select.
__device__ inline void swap_halves2(float x, float y, float& sx, float& sy) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    const auto t = __builtin_amdgcn_permlane32_swap(r[1], r[0], false, false);
    sx = __uint_as_float(t[0]);
    sy = __uint_as_float(t[1]);
}

// Scores, spike tracking, softmax and P.V of one TurboQuant far tile.
template <int D, int NQ, typename QOp>
__device__ inline void tq_far_compute(Lane<D, NQ>& st, const TqTile<D>& r, int tile, int lane, const AttnArgs& a,
                                      const QOp& qr, const QOp& qk, const float (&asum)[NQ]) {
    constexpr int NS = D / 4, NH = D / 64;
    constexpr int KS = NQ == 1 ? 8 : NQ == 2 ? 4 : 2;
    const int blk = lane >> 2;
    const bool general = a.tq_delta != 0.f;
    const PmConst pk = PmConst::make();
    fkv_f4 sh[NQ], sl[NQ], sq[NQ], sx[NQ];
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) sh[qd] = sl[qd] = sq[qd] = sx[qd] = fkv_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s0 = 0; s0 < NS; s0 += KS) {
        fkv_h4 q_r[NQ][KS], q_k[NQ][KS];
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) {
            qr.template readn<KS>(qd, s0, q_r[qd]);
            qk.template readn<KS>(qd, s0, q_k[qd]);
        }
#pragma unroll
        for (int s = s0; s < s0 + KS; s++) {
            const int k = s >> 3, i0 = 2 * (s & 7);
            const fkv_h4 ah = pm1x4(plane_pair(r.kp[0][k]), i0, pk);
            const fkv_h4 al = pm1x4(plane_pair(r.kp[1][k]), i0, pk);
            const fkv_h4 as = pm1x4(plane_pair(r.kp[2][k]), i0, pk);
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) {
                sh[qd] = mfma4_local(ah, q_r[qd][s - s0], sh[qd]);
                sl[qd] = mfma4_local(al, q_r[qd][s - s0], sl[qd]);
                sq[qd] = mfma4_local(as, q_k[qd][s - s0], sq[qd]);
            }
        }
    }
    // The sh*sl term of an asymmetric codebook in a pass of its own, so the
    // common symmetric case takes no branch per k-step.
    if (general) {
#pragma unroll
        for (int s0 = 0; s0 < NS; s0 += KS) {
            fkv_h4 q_r[NQ][KS];
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) qr.template readn<KS>(qd, s0, q_r[qd]);
#pragma unroll
            for (int s = s0; s < s0 + KS; s++) {
                const int k = s >> 3, i0 = 2 * (s & 7);
                const fkv_h4 ax = pm1x4(plane_pair(r.kp[0][k] ^ r.kp[1][k]), i0, pk);
#pragma unroll
                for (int qd = 0; qd < NQ; qd++) sx[qd] = mfma4_local(ax, q_r[qd][s - s0], sx[qd]);
            }
        }
    }
    float p[NQ][4];
    bool any = false;
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = tile * kTile + 4 * blk + e;
            const uint32_t ngw = r.ng[e];
            const float nrm = h2f((uint16_t)(ngw & 0xFFFF)), gmm = h2f((uint16_t)(ngw >> 16));
            float mse = a.tq_beta * sh[qd][e] + a.tq_gamma * sl[qd][e] + asum[qd];
            if (general) mse += a.tq_delta * sx[qd][e];
            const float sv = (nrm * mse + a.tq_qjl * gmm * sq[qd][e]) * a.inv_sqrt_d;
            const bool ok = t < a.L.F;
            sc[e] = ok ? sv : -INFINITY;
            if (ok && sv > st.mx[qd]) { st.mx[qd] = sv; st.arg[qd] = t; }  // first index of the max
        }
        any |= tq_softmax<D, NQ>(st, qd, sc, p[qd]);
    }
    if (__builtin_amdgcn_ballot_w64(any) == 0) return;  // whole tile gated away
    float px[NQ][4];
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
#pragma unroll
        for (int e = 0; e < 4; e += 2) swap_halves2(p[qd][e], p[qd][e + 1], px[qd][e], px[qd][e + 1]);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            p[qd][e] *= a.tq_lvl;
            px[qd][e] *= a.tq_lvl;
        }
    }
#pragma unroll
    for (int dh = 0; dh < NH; dh++) {
        fkv_h4 w[2][NQ];  // [own, other][qd]: p * lvl * the scale of the lane's group 2dh + half
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) {
            _Float16 w0[4], w1[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                w0[e] = (_Float16)(p[qd][e] * half_of(r.so, e * NH + dh));
                w1[e] = (_Float16)(px[qd][e] * half_of(r.sx, e * NH + dh));
            }
            w[0][qd] = fkv_h4{w0[0], w0[1], w0[2], w0[3]};
            w[1][qd] = fkv_h4{w1[0], w1[1], w1[2], w1[3]};
        }
        const uint64_t v[4] = {plane_pair(r.v[dh].x), plane_pair(r.v[dh].y), plane_pair(r.v[dh].z),
                               plane_pair(r.v[dh].w)};
        fkv_f4 po[NQ], pxs[NQ];
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) po[qd] = pxs[qd] = fkv_f4{0.f, 0.f, 0.f, 0.f};
        tq_pv_step<NQ, 0>(po, pxs, v, w, pk);
        tq_pv_step<NQ, 1>(po, pxs, v, w, pk);
        tq_pv_step<NQ, 2>(po, pxs, v, w, pk);
        tq_pv_step<NQ, 3>(po, pxs, v, w, pk);
        tq_pv_step<NQ, 4>(po, pxs, v, w, pk);
        tq_pv_step<NQ, 5>(po, pxs, v, w, pk);
        tq_pv_step<NQ, 6>(po, pxs, v, w, pk);
        tq_pv_step<NQ, 7>(po, pxs, v, w, pk);
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) st.acc[qd][dh] += po[qd] + pxs[qd];
    }
}

// ---------------------------------------------------------------------------
// fp8 K + group-32 INT4 V far tiles (fmt 2)
// ---------------------------------------------------------------------------
//
// Scores as fmt 0.  The value scale / zero change every 32 dims, i.e.
// between the two 32-lane halves of a P.V block, so the scale rides on the
// weights exactly as in the TurboQuant tile: v_mfma_f32_4x4x4_16b_f16 with
// cbsz = 3 gives lanes 0-31 block a's weights (tokens 4a.. of the lanes'
// own half) and lanes 32-63 block 8+a's; a second MFMA takes the other
// half's tokens, whose weights (scaled by this half's group) come across
// with v_permlane32_swap.  The zero point and the +16 decode offset are
// summed per (head, group) and added when the records are written.

template <int D>
constexpr int g32_dma_ops() { return D == 128 ? 13 : 7; }

template <int D>
__device__ inline void dma_g32(const AttnArgs& a, int64_t bkv, int tile, int lane, uint8_t* slot) {
    const uint8_t* rec = a.blob + a.L.far + far_rec_index(a.L, bkv, tile) * (int64_t)a.L.far_rec;
#pragma unroll
    for (int c = 0; c < 3 * D / 32; c++)
        __builtin_amdgcn_global_load_lds((const void*)(rec + c * 1024 + lane * 16), (FKV_LDS void*)(slot + c * 1024), 16,
                                         0, 2);
    // SZ: 8*D bytes = 8*D/16 lanes; for D = 64 the upper lanes repeat the
    // lower lanes' addresses and land past the record in the slot (whole-wave
    // instruction, see dma_tq)
    __builtin_amdgcn_global_load_lds((const void*)(rec + g32_sz_section(D) + (lane & (8 * D / 16 - 1)) * 16),
                                     (FKV_LDS void*)(slot + g32_sz_section(D)), 16, 0, 2);
}

template <int D>
struct FarTileG {
    uint4 k[D / 16];
    uint4 v[D / 32];   // chunk 2*dh + o: o = 0 own half's tokens, 1 the other half's
    uint4 sz[D / 32];  // scale | zero of the lane's 4 tokens, [e][group]
};

__device__ inline void lds_g32(FarTileG<128>& r, const uint8_t* slot, int lane) {
    const uint32_t a = lds_addr(slot + lane * 16), z = lds_addr(slot + g32_sz_section(128) + (lane >> 2) * 64);
    fkv_v4u c[12], zz[4];
    asm volatile(
        "ds_read_b128 %0, %16\n"
        "ds_read_b128 %1, %16 offset:1024\n"
        "ds_read_b128 %2, %16 offset:2048\n"
        "ds_read_b128 %3, %16 offset:3072\n"
        "ds_read_b128 %4, %16 offset:4096\n"
        "ds_read_b128 %5, %16 offset:5120\n"
        "ds_read_b128 %6, %16 offset:6144\n"
        "ds_read_b128 %7, %16 offset:7168\n"
        "ds_read_b128 %8, %16 offset:8192\n"
        "ds_read_b128 %9, %16 offset:9216\n"
        "ds_read_b128 %10, %16 offset:10240\n"
        "ds_read_b128 %11, %16 offset:11264\n"
        "ds_read_b128 %12, %17\n"
        "ds_read_b128 %13, %17 offset:16\n"
        "ds_read_b128 %14, %17 offset:32\n"
        "ds_read_b128 %15, %17 offset:48\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3]), "=&v"(c[4]), "=&v"(c[5]), "=&v"(c[6]), "=&v"(c[7]),
          "=&v"(c[8]), "=&v"(c[9]), "=&v"(c[10]), "=&v"(c[11]), "=&v"(zz[0]), "=&v"(zz[1]), "=&v"(zz[2]),
          "=&v"(zz[3])
        : "v"(a), "v"(z)
        : "memory");
#pragma unroll
    for (int i = 0; i < 8; i++) r.k[i] = u4_of(c[i]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r.v[i] = u4_of(c[8 + i]);
        r.sz[i] = u4_of(zz[i]);
    }
}

__device__ inline void lds_g32(FarTileG<64>& r, const uint8_t* slot, int lane) {
    const uint32_t a = lds_addr(slot + lane * 16), z = lds_addr(slot + g32_sz_section(64) + (lane >> 2) * 32);
    fkv_v4u c[6], zz[2];
    asm volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %8 offset:1024\n"
        "ds_read_b128 %2, %8 offset:2048\n"
        "ds_read_b128 %3, %8 offset:3072\n"
        "ds_read_b128 %4, %8 offset:4096\n"
        "ds_read_b128 %5, %8 offset:5120\n"
        "ds_read_b128 %6, %9\n"
        "ds_read_b128 %7, %9 offset:16\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3]), "=&v"(c[4]), "=&v"(c[5]), "=&v"(zz[0]), "=&v"(zz[1])
        : "v"(a), "v"(z)
        : "memory");
#pragma unroll
    for (int i = 0; i < 4; i++) r.k[i] = u4_of(c[i]);
    r.v[0] = u4_of(c[4]);
    r.v[1] = u4_of(c[5]);
    r.sz[0] = u4_of(zz[0]);
    r.sz[1] = u4_of(zz[1]);
}

// scale | zero word of group g of the lane's token e
__device__ inline uint32_t g32_sz(const uint4* sz, int ng, int e, int g) {
    const int i = e * ng + g;
    return word_of(sz[i >> 2], i & 3);
}

template <int NQ, int A>
__device__ inline void g32_pv_step(fkv_f4& acc0, fkv_f4& acc1, int qd, const uint4 (&v)[4], const fkv_h4& w1a,
                                   const fkv_h4& w2a, const fkv_h4& w1b, const fkv_h4& w2b, bool two) {
    // dh = 0 (chunks 0, 1) and, for D = 128, dh = 1 (chunks 2, 3)
    acc0 = mfma4_half<A>(w1a, int4x4(word_of(v[0], A >> 1), A & 1), acc0);
    if (two) acc1 = mfma4_half<A>(w1b, int4x4(word_of(v[2], A >> 1), A & 1), acc1);
    acc0 = mfma4_half<A>(w2a, int4x4(word_of(v[1], A >> 1), A & 1), acc0);
    if (two) acc1 = mfma4_half<A>(w2b, int4x4(word_of(v[3], A >> 1), A & 1), acc1);
}
// g32_pv_step with the value operands already formed: o[c][A] is chunk c's
// operand of step A.
template <int A>
__device__ inline void g32_pv_step_ops(fkv_f4& acc0, fkv_f4& acc1, const fkv_h4 (&o)[4][8], const fkv_h4& w1a,
                                       const fkv_h4& w2a, const fkv_h4& w1b, const fkv_h4& w2b, bool two) {
    acc0 = mfma4_half<A>(w1a, o[0][A], acc0);
    if (two) acc1 = mfma4_half<A>(w1b, o[2][A], acc1);
    acc0 = mfma4_half<A>(w2a, o[1][A], acc0);
    if (two) acc1 = mfma4_half<A>(w2b, o[3][A], acc1);
}

// Scores, spike tracking, softmax and P.V of one group-32 far tile.
template <int D, int NQ, bool SPK, typename QOp>
__device__ inline void g32_far_compute(Lane<D, NQ>& st, const FarTileG<D>& r, int tile, int F, int lane,
                                       float inv_sqrt_d, const QOp& q_lds, const SpikeTiles& sp) {
    constexpr int NS = D / 4, NH = D / 64, NG = D / 32;
    const int blk = lane >> 2, half = lane >> 5;
    fkv_f4 sacc[NQ];
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) sacc[qd] = fkv_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s0 = 0; s0 < NS; s0 += 8) {
        fkv_h4 q8[NQ][8];
        if constexpr (NQ == 2) {
            q_lds.read8x2(s0, q8);
        } else {
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) q_lds.read8(qd, s0, q8[qd]);
        }
#pragma unroll
        for (int s = s0; s < s0 + 8; s++) {
            const fkv_h4 k4 = e4m3x4(word_of(r.k[s >> 2], s & 3));
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) sacc[qd] = mfma4_local(k4, q8[qd][s - s0], sacc[qd]);
        }
    }
    float p[NQ][4];
    bool any = false;
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = tile * kTile + 4 * blk + e;
            const float sv = sacc[qd][e] * inv_sqrt_d;
            const bool ok = t < F;
            sc[e] = ok ? sv : -INFINITY;
            if (ok && sv > st.mx[qd]) { st.mx[qd] = sv; st.arg[qd] = t; }  // first index of the max
        }
        float cmax = -INFINITY;  // set by the softmax where SPK
        any |= tq_softmax<D, NQ>(st, qd, sc, p[qd], SPK ? &cmax : nullptr);
        store_tile_max<SPK>(sp, qd, tile, cmax);
    }
    if (__builtin_amdgcn_ballot_w64(any) == 0) return;  // whole tile gated away
    // weights: [dh] own-half group (w1) and other-half group before the swap (w2)
    fkv_h4 w1[NH][NQ], w2[NH][NQ];
#pragma unroll
    for (int dh = 0; dh < NH; dh++) {
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) {
            _Float16 a1[4], a2[4];
            float c1[4], c2[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                // group 2dh + half (own) and 2dh + 1 - half (other), selected
                // without a dynamic register index
                const uint32_t za = g32_sz(r.sz, NG, e, 2 * dh), zb = g32_sz(r.sz, NG, e, 2 * dh + 1);
                const uint32_t z1 = half ? zb : za, z2 = half ? za : zb;
                const float s1 = h2f((uint16_t)(z1 & 0xFFFF)), o1 = h2f((uint16_t)(z1 >> 16));
                const float s2 = h2f((uint16_t)(z2 & 0xFFFF)), o2 = h2f((uint16_t)(z2 >> 16));
                a1[e] = (_Float16)(p[qd][e] * s1);
                a2[e] = (_Float16)(p[qd][e] * s2);
                // value = s*(c - 7.5) + (z + 7.5*s) and the MFMA sees w*(16 + c)
                // with w the fp16 weight: the token adds p*(z + 7.5*s) - 23.5*w
                c1[e] = fmaf(-23.5f, (float)a1[e], p[qd][e] * (o1 + 7.5f * s1));
                c2[e] = fmaf(-23.5f, (float)a2[e], p[qd][e] * (o2 + 7.5f * s2));
            }
            st.zsum[qd][dh] += (c1[0] + c1[1]) + (c1[2] + c1[3]);
            st.zsum[qd][NH + dh] += (c2[0] + c2[1]) + (c2[2] + c2[3]);
            w1[dh][qd] = fkv_h4{a1[0], a1[1], a1[2], a1[3]};
            const uint2 x = __builtin_bit_cast(uint2, fkv_h4{a2[0], a2[1], a2[2], a2[3]});
            float y0, y1;
            swap_halves2(__uint_as_float(x.x), __uint_as_float(x.y), y0, y1);
            w2[dh][qd] = __builtin_bit_cast(fkv_h4, make_uint2(__float_as_uint(y0), __float_as_uint(y1)));
        }
    }
    uint4 v4[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v4[i] = r.v[i < NG ? i : 0];
    if constexpr (NQ == 1) {
        // one head quad: every value operand formed before the first MFMA,
        // from dword pairs (words 0, 1 of a chunk serve steps 0-3, words 2, 3
        // steps 4-7)
        fkv_h4 o[4][8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (i >= NG) continue;
            fkv_h4 lo[4], hi[4];
            int4x4_pair(((uint64_t)v4[i].y << 32) | v4[i].x, lo);
            int4x4_pair(((uint64_t)v4[i].w << 32) | v4[i].z, hi);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                o[i][k] = lo[k];
                o[i][4 + k] = hi[k];
            }
        }
        fkv_f4 a0 = st.acc[0][0], a1 = st.acc[0][NH - 1];
        const fkv_h4 w1b = w1[NH - 1][0], w2b = w2[NH - 1][0];
        g32_pv_step_ops<0>(a0, a1, o, w1[0][0], w2[0][0], w1b, w2b, NH == 2);
        g32_pv_step_ops<1>(a0, a1, o, w1[0][0], w2[0][0], w1b, w2b, NH == 2);
        g32_pv_step_ops<2>(a0, a1, o, w1[0][0], w2[0][0], w1b, w2b, NH == 2);
        g32_pv_step_ops<3>(a0, a1, o, w1[0][0], w2[0][0], w1b, w2b, NH == 2);
        g32_pv_step_ops<4>(a0, a1, o, w1[0][0], w2[0][0], w1b, w2b, NH == 2);
        g32_pv_step_ops<5>(a0, a1, o, w1[0][0], w2[0][0], w1b, w2b, NH == 2);
        g32_pv_step_ops<6>(a0, a1, o, w1[0][0], w2[0][0], w1b, w2b, NH == 2);
        g32_pv_step_ops<7>(a0, a1, o, w1[0][0], w2[0][0], w1b, w2b, NH == 2);
        st.acc[0][0] = a0;
        if (NH == 2) st.acc[0][NH - 1] = a1;
        return;
    }
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        fkv_f4 a0 = st.acc[qd][0], a1 = st.acc[qd][NH - 1];
        const fkv_h4 w1b = w1[NH - 1][qd], w2b = w2[NH - 1][qd];
        g32_pv_step<NQ, 0>(a0, a1, qd, v4, w1[0][qd], w2[0][qd], w1b, w2b, NH == 2);
        g32_pv_step<NQ, 1>(a0, a1, qd, v4, w1[0][qd], w2[0][qd], w1b, w2b, NH == 2);
        g32_pv_step<NQ, 2>(a0, a1, qd, v4, w1[0][qd], w2[0][qd], w1b, w2b, NH == 2);
        g32_pv_step<NQ, 3>(a0, a1, qd, v4, w1[0][qd], w2[0][qd], w1b, w2b, NH == 2);
        g32_pv_step<NQ, 4>(a0, a1, qd, v4, w1[0][qd], w2[0][qd], w1b, w2b, NH == 2);
        g32_pv_step<NQ, 5>(a0, a1, qd, v4, w1[0][qd], w2[0][qd], w1b, w2b, NH == 2);
        g32_pv_step<NQ, 6>(a0, a1, qd, v4, w1[0][qd], w2[0][qd], w1b, w2b, NH == 2);
        g32_pv_step<NQ, 7>(a0, a1, qd, v4, w1[0][qd], w2[0][qd], w1b, w2b, NH == 2);
        st.acc[qd][0] = a0;
        if (NH == 2) st.acc[qd][NH - 1] = a1;
    }
}

// Scores, min-near tracking, softmax and P.V of one fp16 tile (near slots or
// decode rows): key operands from kop(s) (lane = token, dims 4s..4s+3),
// value operands from vop(g, dh).
template <int D, int NQ, typename KOp, typename VOp, typename QOp, typename Mid>
__device__ inline void fp16_compute(Lane<D, NQ>& st, KOp kop, VOp vop, int tile, int count, int blk,
                                    float inv_sqrt_d, const QOp& q_lds, Mid after_scores) {
    constexpr int NS = D / 4;
    const QOp qop = q_lds.fresh();
    const uint32_t szd[4] = {0, 0, 0, 0};
    fkv_f4 sacc[NQ];
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) sacc[qd] = fkv_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const fkv_h4 k4 = kop(s);
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) sacc[qd] = mfma4_local(k4, qop(qd, s), sacc[qd]);
    }
    after_scores();
    fkv_h4 w4[NQ];
    bool any = false;
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = tile * kTile + 4 * blk + e;
            const float sv = sacc[qd][e] * inv_sqrt_d;
            const bool ok = t < count;
            sc[e] = ok ? sv : -INFINITY;
            if (ok) st.mn[qd] = fminf(st.mn[qd], sv);
        }
        any |= softmax_w<D, NQ, false>(st, qd, sc, szd, w4[qd]);
    }
    if (__builtin_amdgcn_ballot_w64(any) == 0) return;
    pv_all<D, NQ, 8>(st, w4, vop);
}

// Min-near tracking, softmax and P.V of an fp16 tile whose scores are in
// sacc (token 4*(lane/4) + e, head 4qd + lane%4), value operands from vop.
template <int D, int NQ, typename VOp>
__device__ inline void fp16_pv(Lane<D, NQ>& st, const fkv_f4 (&sacc)[NQ], VOp vop, int tile, int count, int blk,
                               float inv_sqrt_d) {
    const uint32_t szd[4] = {0, 0, 0, 0};
    fkv_h4 w4[NQ];
    bool any = false;
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = tile * kTile + 4 * blk + e;
            const float sv = sacc[qd][e] * inv_sqrt_d;
            const bool ok = t < count;
            sc[e] = ok ? sv : -INFINITY;
            if (ok) st.mn[qd] = fminf(st.mn[qd], sv);
        }
        any |= softmax_w<D, NQ, false>(st, qd, sc, szd, w4[qd]);
    }
    if (__builtin_amdgcn_ballot_w64(any) == 0) return;
    pv_all<D, NQ>(st, w4, vop);
}

// NC 16-byte chunks (1 KB apart) of the lane's operand bytes in an LDS
// slot, read by one asm block that waits for its own LDS reads.
__device__ inline void lds_chunks(fkv_v4u (&o)[16], const uint8_t* p) {
    const uint32_t a = lds_addr(p);
    asm volatile(
        "ds_read_b128 %0, %16\n"
        "ds_read_b128 %1, %16 offset:1024\n"
        "ds_read_b128 %2, %16 offset:2048\n"
        "ds_read_b128 %3, %16 offset:3072\n"
        "ds_read_b128 %4, %16 offset:4096\n"
        "ds_read_b128 %5, %16 offset:5120\n"
        "ds_read_b128 %6, %16 offset:6144\n"
        "ds_read_b128 %7, %16 offset:7168\n"
        "ds_read_b128 %8, %16 offset:8192\n"
        "ds_read_b128 %9, %16 offset:9216\n"
        "ds_read_b128 %10, %16 offset:10240\n"
        "ds_read_b128 %11, %16 offset:11264\n"
        "ds_read_b128 %12, %16 offset:12288\n"
        "ds_read_b128 %13, %16 offset:13312\n"
        "ds_read_b128 %14, %16 offset:14336\n"
        "ds_read_b128 %15, %16 offset:15360\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]), "=&v"(o[7]),
          "=&v"(o[8]), "=&v"(o[9]), "=&v"(o[10]), "=&v"(o[11]), "=&v"(o[12]), "=&v"(o[13]), "=&v"(o[14]),
          "=&v"(o[15])
        : "v"(a)
        : "memory");
}

__device__ inline void lds_chunks(fkv_v4u (&o)[8], const uint8_t* p) {
    const uint32_t a = lds_addr(p);
    asm volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %8 offset:1024\n"
        "ds_read_b128 %2, %8 offset:2048\n"
        "ds_read_b128 %3, %8 offset:3072\n"
        "ds_read_b128 %4, %8 offset:4096\n"
        "ds_read_b128 %5, %8 offset:5120\n"
        "ds_read_b128 %6, %8 offset:6144\n"
        "ds_read_b128 %7, %8 offset:7168\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]), "=&v"(o[7])
        : "v"(a)
        : "memory");
}

// Scores of a near-tier tile whose keys are in an LDS slot (chunk c = dims
// 8c..8c+7 of the lane's token).  With NP parts the slot holds part `part`
// (dims part * D/NP ..); the scores accumulate over the parts, from zero at
// part 0.
template <int D, int NQ, int NP = 1, typename QOp>
__device__ inline void near_scores_lds(fkv_f4 (&sacc)[NQ], const uint8_t* slot, int lane, const QOp& q_lds,
                                       int part = 0) {
    constexpr int NS = D / 4 / NP;
    fkv_v4u kx[D / 8 / NP];
    lds_chunks(kx, slot + lane * 16);
    if (part == 0) {
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) sacc[qd] = fkv_f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int s0 = 0; s0 < NS; s0 += 8) {
        fkv_h4 q8[NQ][8];
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) q_lds.read8(qd, part * NS + s0, q8[qd]);
#pragma unroll
        for (int s = s0; s < s0 + 8; s++) {
            const fkv_v4u& x = kx[s >> 1];
            const fkv_h4 k4 = (s & 1) ? h4_of(x.z, x.w) : h4_of(x.x, x.y);
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) sacc[qd] = mfma4_local(k4, q8[qd][s - s0], sacc[qd]);
        }
    }
}

// Softmax and P.V of a near-tier tile whose values are in an LDS slot
// (8-byte unit x = dh*16 + g of the lane's dim 64dh + lane).
template <int D, int NQ>
__device__ inline void near_pv_lds(Lane<D, NQ>& st, const fkv_f4 (&sacc)[NQ], const uint8_t* slot, int lane,
                                   int tile, int count, float inv_sqrt_d) {
    fkv_v4u vx[D / 8];
    lds_chunks(vx, slot + lane * 16);
    fp16_pv<D, NQ>(
        st, sacc,
        [&](int g, int dh) {
            const int xi = dh * 16 + g;
            const fkv_v4u& x = vx[xi >> 1];
            return (xi & 1) ? h4_of(x.z, x.w) : h4_of(x.x, x.y);
        },
        tile, count, lane >> 2, inv_sqrt_d);
}

// The same over D = 128 values split in two parts (dim halves dh = 0, 1,
// one ring slot each): part 0 runs the softmax and keeps the weights in w4
// (and whether any is non-zero in `any`) for part 1.
template <int D, int NQ, int G>
__device__ inline void pv_group_dh(Lane<D, NQ>& st, const fkv_h4 (&w4)[NQ], const fkv_v4u (&vx)[8], int dh) {
    const fkv_v4u& x = vx[G >> 1];
    const fkv_h4 v = (G & 1) ? h4_of(x.z, x.w) : h4_of(x.x, x.y);
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) st.acc[qd][dh] = mfma4<G>(w4[qd], v, st.acc[qd][dh]);
}

template <int D, int NQ, int PART>
__device__ inline void near_pv_lds_part(Lane<D, NQ>& st, const fkv_f4 (&sacc)[NQ], fkv_h4 (&w4)[NQ], bool& any,
                                        const uint8_t* slot, int lane, int tile, int count, float inv_sqrt_d) {
    constexpr int part = PART;
    static_assert(D == 128, "two value parts are one 64-dim half each");
    fkv_v4u vx[8];
    lds_chunks(vx, slot + lane * 16);
    if constexpr (part == 0) {
        const uint32_t szd[4] = {0, 0, 0, 0};
        const int blk = lane >> 2;
        any = false;
#pragma unroll
        for (int qd = 0; qd < NQ; qd++) {
            float sc[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = tile * kTile + 4 * blk + e;
                const float sv = sacc[qd][e] * inv_sqrt_d;
                const bool ok = t < count;
                sc[e] = ok ? sv : -INFINITY;
                if (ok) st.mn[qd] = fminf(st.mn[qd], sv);
            }
            any |= softmax_w<D, NQ, false>(st, qd, sc, szd, w4[qd]);
        }
    }
    if (__builtin_amdgcn_ballot_w64(any) == 0) return;
    pv_group_dh<D, NQ, 0>(st, w4, vx, part);
    pv_group_dh<D, NQ, 1>(st, w4, vx, part);
    pv_group_dh<D, NQ, 2>(st, w4, vx, part);
    pv_group_dh<D, NQ, 3>(st, w4, vx, part);
    pv_group_dh<D, NQ, 4>(st, w4, vx, part);
    pv_group_dh<D, NQ, 5>(st, w4, vx, part);
    pv_group_dh<D, NQ, 6>(st, w4, vx, part);
    pv_group_dh<D, NQ, 7>(st, w4, vx, part);
    pv_group_dh<D, NQ, 8>(st, w4, vx, part);
    pv_group_dh<D, NQ, 9>(st, w4, vx, part);
    pv_group_dh<D, NQ, 10>(st, w4, vx, part);
    pv_group_dh<D, NQ, 11>(st, w4, vx, part);
    pv_group_dh<D, NQ, 12>(st, w4, vx, part);
    pv_group_dh<D, NQ, 13>(st, w4, vx, part);
    pv_group_dh<D, NQ, 14>(st, w4, vx, part);
    pv_group_dh<D, NQ, 15>(st, w4, vx, part);
}

// Decode-buffer tile: rows (n_dec, D) row-major fp16.  The tile's value
// rows are copied into `stage` (the wave's idle ring, 2 * 64 * D bytes, row
// t at byte 2 D t) by LDS DMA first, rows past `count` repeating the last
// row (finite values that meet weight 0); then a lane reads its token's key
// row for the score operand, so the two loads share one round trip; the
// value operand (dim 64dh + lane of the 4 tokens of group g) is read from
// the stage once the scores are done.
template <int D, int NQ, typename QOp>
__device__ inline void dec_tile(Lane<D, NQ>& st, const AttnArgs& a, int count, int64_t bkv, int tile, int lane,
                                const QOp& qop, uint8_t* stage) {
    constexpr int CPR = D / 8;                // 16-byte chunks of a row
    constexpr int NI = kTile * CPR / kWave;  // DMA instructions of the tile
    const int rows = min(count - tile * kTile, kTile);
    const uint16_t* vt = a.dec_v + (bkv * a.dec_stride + (int64_t)tile * kTile) * D;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c = i * kWave + lane, t = c / CPR;
        __builtin_amdgcn_global_load_lds((const void*)(vt + (int64_t)(t < rows ? t : rows - 1) * D + (c % CPR) * 8),
                                         (FKV_LDS void*)(stage + i * 1024), 16, 0, 0);
    }
    const int tk = tile * kTile + lane;
    uint4 kx[D / 8];
    const bool kin = tk < count;
    const uint16_t* kr = a.dec_k + (bkv * a.dec_stride + (kin ? tk : 0)) * D;  // a valid row: no branch per load
#pragma unroll
    for (int c = 0; c < D / 8; c++) {
        const uint4 x = *(const uint4*)(kr + c * 8);
        kx[c] = kin ? x : make_uint4(0, 0, 0, 0);
    }
    const uint16_t* vs = (const uint16_t*)stage + lane;
    fp16_compute<D, NQ>(
        st,
        [&](int s) {
            const uint4& x = kx[s >> 1];
            return (s & 1) ? h4_of(x.z, x.w) : h4_of(x.x, x.y);
        },
        [&](int g, int dh) {
            const uint16_t* p = vs + 4 * g * D + 64 * dh;
            return h4_of(p[0] | ((uint32_t)p[D] << 16), p[2 * D] | ((uint32_t)p[3 * D] << 16));
        },
        tile, count, lane >> 2, a.inv_sqrt_d, qop,
        // the compiler does not order LDS reads after the DMA
        []() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); });
}

// The XCD this wave runs on.
__device__ inline uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 0xF;
}

// Merge of the partial records of all splits of one row
// (csrc/kernels/foveated_attn.metal:394-431 restated for partials in
// memory): split maxima are rescaled to the global max; spike fields take
// the min and the first-index max.
//
// Loads of split records: buffer loads with the sc1 cache policy (the
// policy of agent-scope atomic loads: coherent across XCDs) or, where every
// split of the row ran on one XCD (xcd_mod), sc0 (past the CU's L1, served
// by the XCD's L2); offsets past the buffer read 0 without touching memory.
constexpr int kCpolSc1 = 16, kCpolSc0 = 1;
template <int CPOL>
__device__ inline fkv_f4 ld_rec4(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(fkv_f4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, CPOL));
}
template <int CPOL>
__device__ inline int ld_rec1(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, CPOL);
}

// 64-lane reductions on DPP row rotations and lane swaps (no LDS permutes):
// max / min / (max, first index) reach every lane; the sum is a fixed tree
// whose lanes may round differently, so lane 0's value is returned.
__device__ inline float wave_max_dpp(float v) {
    v = fmaxf(v, __uint_as_float(row_ror<1>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(row_ror<2>(__float_as_uint(v))));
    return head_max(v);
}
__device__ inline float wave_min_dpp(float v) {
    v = fminf(v, __uint_as_float(row_ror<1>(__float_as_uint(v))));
    v = fminf(v, __uint_as_float(row_ror<2>(__float_as_uint(v))));
    return head_min(v);
}
__device__ inline float wave_sum_dpp(float v) {
    v += __uint_as_float(row_ror<1>(__float_as_uint(v)));
    v += __uint_as_float(row_ror<2>(__float_as_uint(v)));
    return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(head_sum<true>(v))));
}
__device__ inline void wave_argmax_dpp(float& mx, int& arg) {
    pick_max(mx, arg, __uint_as_float(row_ror<1>(__float_as_uint(mx))), (int)row_ror<1>((uint32_t)arg));
    pick_max(mx, arg, __uint_as_float(row_ror<2>(__float_as_uint(mx))), (int)row_ror<2>((uint32_t)arg));
    head_argmax(mx, arg);
}

// Reductions over the 16 lanes of each row (DPP rotations only); lanes of
// row 0 hold the result for lanes 0-15.
__device__ inline float row_max16(float v) {
    v = fmaxf(v, __uint_as_float(row_ror<1>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(row_ror<2>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(row_ror<4>(__float_as_uint(v))));
    return fmaxf(v, __uint_as_float(row_ror<8>(__float_as_uint(v))));
}
__device__ inline float row_min16(float v) {
    v = fminf(v, __uint_as_float(row_ror<1>(__float_as_uint(v))));
    v = fminf(v, __uint_as_float(row_ror<2>(__float_as_uint(v))));
    v = fminf(v, __uint_as_float(row_ror<4>(__float_as_uint(v))));
    return fminf(v, __uint_as_float(row_ror<8>(__float_as_uint(v))));
}
__device__ inline float row_sum16(float v) {
    v += __uint_as_float(row_ror<1>(__float_as_uint(v)));
    v += __uint_as_float(row_ror<2>(__float_as_uint(v)));
    v += __uint_as_float(row_ror<4>(__float_as_uint(v)));
    return v + __uint_as_float(row_ror<8>(__float_as_uint(v)));
}
__device__ inline void row_argmax16(float& mx, int& arg) {
    pick_max(mx, arg, __uint_as_float(row_ror<1>(__float_as_uint(mx))), (int)row_ror<1>((uint32_t)arg));
    pick_max(mx, arg, __uint_as_float(row_ror<2>(__float_as_uint(mx))), (int)row_ror<2>((uint32_t)arg));
    pick_max(mx, arg, __uint_as_float(row_ror<4>(__float_as_uint(mx))), (int)row_ror<4>((uint32_t)arg));
    pick_max(mx, arg, __uint_as_float(row_ror<8>(__float_as_uint(mx))), (int)row_ror<8>((uint32_t)arg));
}

// Spike fields (lane 0) and the merged output of one head: value lane
// (c, u) accumulates its splits u, u + SUB, ... in order, with each split's
// scale read from that split's lane; the SUB lane groups combine by lane
// swaps; lanes of group 0 write chunk c.
template <int D, int NH, int KV, bool EXT>
__device__ inline void merge_values(const AttnArgs& a, const fkv_f4 (&v)[KV], float f, float M, float L, float mn,
                                    float mx, int arg, int nk, int u, int c, int lane, int64_t o) {
    constexpr int SUB = kWave / (D / 4);
    (void)M;
    if (lane == 0) {
        a.flags[o] = mx > mn + a.spike_margin ? 1 : 0;
        a.tokens[o] = mx == -INFINITY ? -1 : arg;
        if (EXT && a.thr) a.thr[o] = mn + a.spike_margin;
    }
    // in the load groups of 4: splits past the last have scale 0 and value 0
    fkv_f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k0 = 0; k0 < KV; k0 += 4) {
        if (k0 < nk) {
#pragma unroll
            for (int k = k0; k < k0 + 4 && k < KV; k++) {
                float fs = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), SUB * k));
#pragma unroll
                for (int uu = 1; uu < SUB; uu++) {
                    const float fu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), SUB * k + uu));
                    fs = u == uu ? fu : fs;
                }
                acc.x = fmaf(fs, v[k].x, acc.x);
                acc.y = fmaf(fs, v[k].y, acc.y);
                acc.z = fmaf(fs, v[k].z, acc.z);
                acc.w = fmaf(fs, v[k].w, acc.w);
            }
        }
    }
    if (SUB == 4) {
        LanePair px = swap16(__float_as_uint(acc.x)), py = swap16(__float_as_uint(acc.y));
        LanePair pz = swap16(__float_as_uint(acc.z)), pw = swap16(__float_as_uint(acc.w));
        acc = fkv_f4{__uint_as_float(px.a) + __uint_as_float(px.b), __uint_as_float(py.a) + __uint_as_float(py.b),
                     __uint_as_float(pz.a) + __uint_as_float(pz.b), __uint_as_float(pw.a) + __uint_as_float(pw.b)};
    }
    {
        LanePair px = swap32(__float_as_uint(acc.x)), py = swap32(__float_as_uint(acc.y));
        LanePair pz = swap32(__float_as_uint(acc.z)), pw = swap32(__float_as_uint(acc.w));
        acc = fkv_f4{__uint_as_float(px.a) + __uint_as_float(px.b), __uint_as_float(py.a) + __uint_as_float(py.b),
                     __uint_as_float(pz.a) + __uint_as_float(pz.b), __uint_as_float(pw.a) + __uint_as_float(pw.b)};
    }
    if (u == 0) {
        const float il = L > 0.f ? 1.0f / L : 0.f;
        const uint2 w = {f2h(acc.x * il) | ((uint32_t)f2h(acc.y * il) << 16),
                         f2h(acc.z * il) | ((uint32_t)f2h(acc.w * il) << 16)};
        *(uint2*)(a.out + o * D + 4 * c) = w;
    }
}

// Split records of NH heads (g0, g0 + step, ...) of one row merged by one
// wave.  Lane s reads split s's header; lane (c, u) = (lane % CH, lane /
// CH) reads value chunk c (4 dims) of the splits u, u + SUB, u + 2 SUB, ...
// Every load of the NH heads is issued before the first wait.  The split
// maxima, sums, minima and first-index maxima reduce on DPP; each value lane
// accumulates its splits in order with the split scales read from the
// scale's lane, and the SUB lane groups combine by lane swaps.  The
// in-kernel merge and merge_kernel both run this, so both give the same
// bits.  Needs nk = ceil(ns / SUB) <= KV / NH.
template <int D, int NH>
constexpr int merge_kv() { return kMaxSplits / (kWave / (D / 4)) / NH; }  // value loads per lane and head

// The record loads of merge_heads with cache policy CPOL.
template <int D, int NH, int CPOL>
__device__ inline void merge_loads(__amdgpu_buffer_rsrc_t rs, int ng, int nk, int g0, int step, int lane,
                                   fkv_f4 (&h)[NH], int (&harg)[NH], uint32_t (&hx)[NH],
                                   fkv_f4 (&v)[NH][merge_kv<D, NH>()]) {
    constexpr int RS = kHdr + D;
    constexpr int CH = D / 4, SUB = kWave / CH;
    const int c = lane % CH, u = lane / CH;
    const int sstride = ng * RS * 4;  // bytes from one split's record to the next
#pragma unroll
    for (int i = 0; i < NH; i++) {
        const int g = g0 + i * step;
        const int hoff = lane * sstride + g * RS * 4;
        h[i] = ld_rec4<CPOL>(rs, hoff);
        // header words 4, 5: the first-index argmax and the writer's XCD
        const fkv_v2u ax = __builtin_bit_cast(fkv_v2u, __builtin_amdgcn_raw_buffer_load_b64(rs, hoff + 16, 0, CPOL));
        harg[i] = (int)ax.x;
        hx[i] = ax.y;
        const int voff = u * sstride + (g * RS + kHdr + 4 * c) * 4;
        // in groups of 4 behind one branch: loads past the last split read
        // 0 without touching memory (and meet scale 0)
#pragma unroll
        for (int k0 = 0; k0 < merge_kv<D, NH>(); k0 += 4)
            if (k0 < nk)
#pragma unroll
                for (int k = k0; k < k0 + 4 && k < merge_kv<D, NH>(); k++)
                    v[i][k] = __builtin_bit_cast(
                        fkv_f4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, SUB * k * sstride, CPOL));
    }
}

template <int D, int NH, bool EXT = false>
__device__ inline void merge_heads(const AttnArgs& a, __amdgpu_buffer_rsrc_t rs, int ns, int ng, int g0, int step,
                                   int lane, int64_t o0, bool xcd_local = false) {
    constexpr int CH = D / 4;          // 16-byte value chunks of a head
    constexpr int SUB = kWave / CH;    // lane groups over the splits
    constexpr int KV = merge_kv<D, NH>();
    const int c = lane % CH, u = lane / CH;
    const int nk = (ns + SUB - 1) / SUB;
    // Offsets past the last record read 0 without touching memory: lanes
    // past ns are masked below, value loads of splits past ns meet scale 0.
    fkv_f4 h[NH];
    int harg[NH];
    uint32_t hx[NH];
    fkv_f4 v[NH][KV];
    if (xcd_local) merge_loads<D, NH, kCpolSc0>(rs, ng, nk, g0, step, lane, h, harg, hx, v);
    else merge_loads<D, NH, kCpolSc1>(rs, ng, nk, g0, step, lane, h, harg, hx, v);
    const bool live = lane < ns;
    // XCD-local merge: every split record of the row must come from this
    // XCD (the dispatch rule); one from another XCD -- or a stale one a
    // split left in another L2 -- means this merge may have read stale
    // records, and raises the handle's watch flag for the host
    if (xcd_local) {
        const uint32_t me = xcc_id();
        bool other = false;
#pragma unroll
        for (int i = 0; i < NH; i++) other |= live && hx[i] != me;
        if (__builtin_amdgcn_ballot_w64(other) != 0 && lane == 0)
            __hip_atomic_fetch_or(a.xcd_watch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const bool one_row = ns <= 16;  // the live lanes sit in the first 16: row reductions suffice
#pragma unroll
    for (int i = 0; i < NH; i++) {
        const float ms = live ? h[i].x : -INFINITY;
        float mn = live ? h[i].z : INFINITY, mx = live ? h[i].w : -INFINITY;
        int arg = live ? harg[i] : INT_MAX;
        float M, L;
        if (one_row) {
            M = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(row_max16(ms))));
            const float f = ms == -INFINITY ? 0.f : __expf(ms - M);  // 0 past the last split
            L = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(row_sum16(live ? f * h[i].y : 0.f))));
            mn = row_min16(mn);
            row_argmax16(mx, arg);
            merge_values<D, NH, KV, EXT>(a, v[i], f, M, L, mn, mx, arg, nk, u, c, lane, o0 + i * step);
        } else {
            M = wave_max_dpp(ms);
            const float f = ms == -INFINITY ? 0.f : __expf(ms - M);
            L = wave_sum_dpp(live ? f * h[i].y : 0.f);
            mn = wave_min_dpp(mn);
            wave_argmax_dpp(mx, arg);
            merge_values<D, NH, KV, EXT>(a, v[i], f, M, L, mn, mx, arg, nk, u, c, lane, o0 + i * step);
        }
    }
}

// XCD-local merge.  The command processor deals a dispatch's workgroups to
// the X XCDs round-robin by linear workgroup index: index i runs on XCD
// (c + i) mod X, with an offset c that is fixed for the dispatch (it
// differs between hardware queues).  The host checks this rule once per
// device (xcd_rule; a handle created with FKV_XCD_LOCAL=0 in the
// environment does not use it).  Where a launch's rows are a multiple of X
// the kernel numbers its workgroups split-major (i = split * rows + row),
// so every split of a row runs on XCD (c + row) mod X whatever c is, and
// the row's records, counter and merge stay in that XCD's L2: records are
// written with plain stores (to L2), the arrival is an L2 atomic, the last
// split reads the records with sc0 loads (past its L1).  Otherwise (and for
// launches with one split) the merge is coherent across XCDs (sc1 and
// agent scope), as described at the merged-record publish.

// One workgroup's arrival at its row; true for the row's last split.
__device__ inline bool arrive_last(const AttnArgs& a, int row, bool xcd_local) {
    const int prev = xcd_local ? __hip_atomic_fetch_add(a.arrive + row, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                               : __hip_atomic_fetch_add(a.arrive + row, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return prev == a.num_splits - 1;
}
// The last split re-arms the row's counter for the next launch.
__device__ inline void rearm(const AttnArgs& a, int row, bool xcd_local) {
    if (xcd_local) __hip_atomic_store(a.arrive + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else __hip_atomic_store(a.arrive + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The last split of a row merges every split's record: wave w of the WPG
// takes heads w, w + WPG, ... (two at a time where their loads fit the
// registers).
template <int D, int WPG = kWavesPerGroup, bool EXT = false>
__device__ inline void merge_finalize_direct(const AttnArgs& a, const float* src, int ns, int ng, int b, int head0,
                                             bool xcd_local, int row) {
    constexpr int RS = kHdr + D;
    (void)row;
    constexpr int SUB = kWave / (D / 4);
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave), lane = (int)threadIdx.x % kWave;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, ns * ng * RS * 4, 0x00020000);
    const int hw = wave < ng ? (ng - wave + WPG - 1) / WPG : 0;  // this wave's heads
    const int nk = (ns + SUB - 1) / SUB;
    const int64_t o0 = (int64_t)b * a.Hq + head0 + wave;
    int j = 0;
    if (hw >= 2 && nk <= kMaxSplits / SUB / 2) {
        merge_heads<D, 2, EXT>(a, rs, ns, ng, wave, WPG, lane, o0, xcd_local);
        j = 2;
    }
    for (; j < hw; j++) merge_heads<D, 1, EXT>(a, rs, ns, ng, wave + j * WPG, WPG, lane, o0 + j * WPG, xcd_local);
}

// Unit u of one wave's stream: the wave's far tiles first (far tile
// f0 + u*fs), then each of its near tiles w + j*N as 2 * NP units: the keys
// in NP parts of D / NP dims, then the values in NP parts of D / NP dims
// (NP = 2 keeps every unit within an 8 KB ring slot at D = 128).  w is the
// wave's index among the N waves of its row.
enum UnitKind { kNone = 0, kFarUnit = 1, kNearK = 2, kNearV = 3 };
template <int NP>
struct Units {
    int w, N, f0, fs, nf, nn;
    int wn;  // the wave's place in the near-tile deal: near tiles wn, wn + N, ...
    __device__ int count() const { return nf + 2 * NP * nn; }
    __device__ int kind(int u) const {
        return u >= nf + 2 * NP * nn ? kNone : u < nf ? kFarUnit : (u - nf) % (2 * NP) < NP ? kNearK : kNearV;
    }
    __device__ int part(int u) const { return (u - nf) % NP; }
    __device__ int tile(int u) const { return u < nf ? f0 + u * fs : wn + (u - nf) / (2 * NP) * N; }
};


// Far tiles of wave w of a row, balanced against the row's near tiles
// (near tile t goes to wave t mod N; `near_plan` is the host's expected near
// tile count, so the split needs no device read; a near tile weighs NB, a
// far tile its record bytes FB): contiguous ranges whose boundaries round
// v / N of the row's weight minus the near weight before wave v, clamped to
// [0, F].  The unclamped boundary is linear in v with a
// positive slope once v passes the waves with an extra near tile and passes
// through 0 before, so the clamped boundaries never decrease; waves holding
// more near tiles than their share take no far tiles.  TurboQuant far tiles
// cost far more time per byte than near tiles, so where a wave's far share is
// below one near tile they are dealt round-robin instead.  The host repeats
// this plan (far_bound) to place decode tiles.
struct FarPlan {
    int f0, fs, nf;
};

__host__ __device__ inline int far_bound(int64_t v, int64_t N, int NT, int FT, int64_t NB, int64_t FB) {
    if (v >= N) return FT;
    const int64_t q = NT / N, r = NT % N;
    const int64_t total = NT * NB + (int64_t)FT * FB;
    const int64_t near_before = v * q + (v < r ? v : r);
    const int64_t num = v * total - N * near_before * NB;
    const int64_t g = (2 * num + N * FB) / (2 * N * FB);  // round to nearest (negative: clamped)
    return (int)(g < 0 ? 0 : g > FT ? FT : g);
}

__host__ __device__ inline bool far_round_robin(bool tq, int64_t N, int FT, int64_t NB, int64_t FB) {
    return tq && (int64_t)FT * FB < N * NB;
}
// Where the near-tile deal starts: wave 0, or, where far tiles are dealt
// round-robin (waves from FT mod N on hold one far tile fewer), at FT mod N,
// so the near tiles go to those waves first.  The host starts decode tiles
// after the near tiles with the same rule.
__host__ __device__ inline int near_deal_start(bool tq, int64_t N, int FT, int64_t NB, int64_t FB) {
    return far_round_robin(tq, N, FT, NB, FB) ? (int)(FT % N) : 0;
}

// The weight of a near tile in the far split, in bytes: its K and V bytes
// (256 * D) where the stream is bound by HBM (one head quad); half of that
// for 8-16 query heads per row, whose far tiles cost more arithmetic per
// byte than the fp16 near tiles (measured: C5, 64K, G = 8, 42.6 -> 40.0 us).
__host__ __device__ inline int64_t near_tile_weight(int nq, int D) { return (nq >= 2 ? 128 : 256) * (int64_t)D; }

__host__ __device__ inline FarPlan plan_far(int w, int n_waves, int nt_far, int near_plan, int64_t FB, bool tq,
                                            int64_t NB) {
    if (!far_round_robin(tq, n_waves, nt_far, NB, FB)) {
        const int f0 = far_bound(w, n_waves, near_plan, nt_far, NB, FB);
        return FarPlan{f0, 1, far_bound(w + 1, n_waves, near_plan, nt_far, NB, FB) - f0};
    }
    return FarPlan{w, n_waves, w < nt_far ? (int)cdiv(nt_far - w, n_waves) : 0};
}

// TurboQuant query rotation and sketch inside the attention kernel:
// q.Pi^T and q.S^T (foveated_attn.cpp:415-421) for the workgroup's heads on
// the matrix cores.  Wave w < D/32 takes matrix mat and the 64 output dims
// 64 * rg .. + 63 (lane l: output dim 64 * rg + l as the A row of
// v_mfma_f32_4x4x4f16, the head quad's fp16 query as B) with M in fp16
// (tq_rot_index), one accumulator chain over the D/4 k-steps.  The products
// of fp16 values are exact and summed in fp32; M's own fp16 rounding adds
// at most about as much as the final rounding of the rotated query to fp16
// (a lo correction, M - fp16(M), in a second chain had cost C4 1.1 us of
// operand loads and matrix instructions for no visible parity change: C4
// max-abs 1.6e-4 either way).  Lane l ends with
// dims 64 * rg + 4 * (l / 4) .. + 3 of head l % 4, rounded to fp16 into the
// qt operand layout; mat 0 also leaves q.Pi^T in fp32 in `qf` and alpha *
// sum(q.Pi^T) per head in `rsum`.  Waves past D/32 only take part in the
// barriers.  Must be entered by every thread of the workgroup.
template <int D>
struct TqRotation {
    fkv_v4u h[D / 8];  // [s2]: k-steps 2 * s2, 2 * s2 + 1 of the lane's row
};

// The wave's A operands, loaded together with the query (before any use);
// waves past D/32 load nothing.
template <int D, int WPG>
__device__ inline void tq_rotation_load(const AttnArgs& a, TqRotation<D>& r, int wave, int lane) {
    constexpr int WR = D / 32, RG = D / 64;
    if (wave >= WR) return;
    const int wr = wave % WR, mat = wr / RG, rg = wr % RG;
#pragma unroll
    for (int s2 = 0; s2 < D / 8; s2++)
        r.h[s2] = *(const fkv_v4u*)(a.tq_rot + tq_rot_index(D, mat, 64 * rg + lane, 8 * s2));
}

template <int D, int NQ, int WPG>
__device__ inline void tq_rotate_query(const AttnArgs& a, const TqRotation<D>& rot, const QOperand<D / 4>& qop,
                                       float* qf, uint16_t* qt, float* rsum, int wave, int lane) {
    constexpr int NS = D / 4, WR = D / 32, RG = D / 64;
    const int wr = wave % WR, mat = wr / RG, rg = wr % RG;
    const int c = lane & 3, blk = lane >> 2;
    const bool idle = wave >= WR;  // no operands loaded
#pragma unroll 1
    for (int qd = 0; qd < NQ && !idle; qd++) {
        fkv_f4 ch = fkv_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s0 = 0; s0 < NS; s0 += 8) {
            fkv_h4 q8[8];
            qop.template readn<8>(qd, s0, q8);
#pragma unroll
            for (int s = s0; s < s0 + 8; s++) {
                const fkv_v4u& h = rot.h[s / 2];
                const fkv_h4 ah = __builtin_bit_cast(fkv_h4, (s & 1) ? fkv_v2u{h.z, h.w} : fkv_v2u{h.x, h.y});
                ch = mfma4_local(ah, q8[s - s0], ch);
            }
        }
        if (wave < WR) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = ch[e];
            const int sq = 16 * rg + blk;  // k-step of output dims 4 * sq .. 4 * sq + 3
            const uint32_t w0 = (uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16);
            const uint32_t w1 = (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16);
            *(fkv_v2u*)(qt + mat * NQ * NS * 16 + ((qd * NS + sq) * 4 + c) * 4) = fkv_v2u{w0, w1};
            if (mat == 0) *(float4*)(qf + (4 * qd + c) * D + 4 * sq) = float4{v[0], v[1], v[2], v[3]};
        }
    }
    if (a.tq_alpha != 0.f) {
        lds_barrier();
        // wave w sums head w's rotated query of every quad
        if (wave < 4) {
            for (int qd = 0; qd < NQ; qd++) {
                float v = 0.f;
                for (int col = lane; col < D; col += kWave) v += qf[(4 * qd + wave) * D + col];
                v = wave_sum(v);
                if (lane == 0) rsum[4 * qd + wave] = a.tq_alpha * v;
            }
        }
    }
    lds_barrier();
}

// One workgroup of 4 waves (8: attn_waves) per (batch, kv head, split, head
// group); each wave streams its units through a 2-slot LDS ring with
// gfx950's direct global->LDS loads: the next unit's bytes stream in while
// the current one is computed.  The ring takes most of the CU's LDS (one
// workgroup per CU).
// EXT: the kernel of handles that use an extension beyond the reference --
// per-head-scaled fp8 keys (a.kscale, chosen at run time) or top-K spike
// tokens; SPK (top-K handles only, implies EXT): the far tiles also store
// their per-head maxima (a.tmax) and the merge the heads' thresholds
// (a.thr).  Without EXT none of it exists and the reference's path keeps
// its registers; each kernel has one far-tile body (a run-time choice
// between two bodies in the stream loop had cost the extension kernels
// ~1.2 us at C5 even where they took the plain one).
template <int D, int NQ, int FMT, bool EXT = false, bool SPK = false>
__global__ __launch_bounds__(64 * attn_waves(D, NQ, FMT)) void attn_kernel(AttnArgs a) {
    static_assert(EXT || !SPK, "the top-K kernels are extension kernels");
    constexpr int WPG = attn_waves(D, NQ, FMT);  // waves of the workgroup
    constexpr int NS = D / 4;   // 4-dim k-steps of QK
    constexpr int NH = D / 64;  // 64-dim halves of P.V
    constexpr int RS = kHdr + D;
    constexpr int NHW = 4 * NQ;  // head records per wave
    constexpr bool TQ = FMT == 1, G32 = FMT == 2;
    constexpr int REC = (int)(TQ ? tq_record_bytes(D) : G32 ? g32_record_bytes(D) : far_record_bytes(D));
    // near K / V halves in NP parts: TurboQuant at D = 128 streams 8 KB units
    // (its 64 KB ring lets two workgroups share a CU)
    constexpr int NP = TQ && D == 128 ? 2 : 1;
    constexpr int SLOT = REC > 128 * D / NP ? REC : 128 * D / NP;  // far record or a near K / V part
    constexpr int FAR_OPS = TQ ? tq_dma_ops<D>() : G32 ? g32_dma_ops<D>() : far_dma_ops<D>(), NEAR_OPS = D / 8 / NP;
    static_assert(FAR_OPS != NEAR_OPS, "the ring's vmcnt waits tell far and near units apart by op count");
    // the query as score operands: one copy per wave (each wave stages its
    // own by LDS DMA and waits for nothing but its own loads), one shared
    // copy for TurboQuant (staged by all threads behind a barrier)
    constexpr int QCOPY = NQ * NS * 4 * 4, NQC = TQ ? 1 : WPG;
    __shared__ __attribute__((aligned(16))) uint16_t qs[NQC * QCOPY];
    // TurboQuant: rotated and sketched query operands, same layout as qs;
    // the fp32 query and the per-head alpha * sum(q.Pi^T)
    __shared__ __attribute__((aligned(16))) uint16_t qt[TQ ? 2 * NQ * NS * 4 * 4 : 8];
    __shared__ __attribute__((aligned(16))) float qf[TQ ? 4 * NQ * D : 4];
    __shared__ float rsum[TQ ? 4 * NQ : 4];
    // The rings during the tile loop, and the per-wave records merged in LDS
    // after it: past the rings where both fit the CU's 160 KB (a wave then
    // writes its record as soon as its own stream ends), else over them
    // (behind a barrier once every wave's stream has ended).
    constexpr int kRing = WPG * 2 * SLOT;
    static_assert(2 * SLOT >= kTile * D * 2, "a wave's ring holds a decode tile's value rows");
    constexpr int kRec = WPG * NHW * RS * 4;
    constexpr int kQ = 2 * NQC * QCOPY + (TQ ? 4 * NQ * NS * 16 + 16 * NQ * D + 16 * NQ : 64);
    constexpr bool SEP_REC = kRing + kRec + kQ + 256 <= 160 * 1024;
    constexpr int kLds = SEP_REC ? kRing + kRec : (kRing > kRec ? kRing : kRec);
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
    float* smem = (float*)(lds + (SEP_REC ? kRing : 0));
    __shared__ int s_last;

    // XCD-local merge: linear workgroup index = split * rows + row, so that
    // every split of a row runs on one XCD (rows is a multiple of xcd_mod)
    const bool xcd_local = a.xcd_mod != 0;
    int split = blockIdx.x, rowl = blockIdx.y + gridDim.y * blockIdx.z;
    if (xcd_local) {
        const int rows = gridDim.y * gridDim.z, lin = blockIdx.x + gridDim.x * rowl;
        split = lin / rows;
        rowl = lin % rows;
    }
    const int kvh = (rowl % gridDim.y) / a.head_groups;
    const int hgrp = (rowl % gridDim.y) % a.head_groups;
    const int b = rowl / gridDim.y;
    const int64_t bkv = (int64_t)b * a.L.Hkv + kvh;
    const int head0 = kvh * a.G + hgrp * a.hpg;
    const int ng = min(a.hpg, a.G - hgrp * a.hpg);
    FKV_STAMP_AT(threadIdx.x == 0, 0);
#ifdef FKV_PHASE_STAMPS
    if (threadIdx.x == 0) {
        const int wg_ = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
        if (wg_ < kStampWGs) a.stamps[kStampSlots * wg_ + kStampSlots - 1] = xcc_id();
    }
#endif
    // the wave index is wave-uniform: scalar registers, scalar branches
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave), lane = threadIdx.x % kWave;
    const int j = lane & 3, blk = lane >> 2;
    uint8_t* ring = lds + wave * 2 * SLOT;

    // ---- the wave's far tiles need no device state: start streaming ----
    Units<NP> un;
    un.N = WPG * a.num_splits;
    // TurboQuant deals its far and near tiles round-robin over the row's
    // waves (far_round_robin): numbered wave-major, so that consecutive tiles
    // go to different workgroups and every workgroup gets an equal share
    un.w = TQ ? wave * a.num_splits + split : WPG * split + wave;
    {
        const FarPlan fp =
            plan_far(un.w, un.N, (int)cdiv(a.L.F, kTile), a.near_plan, REC, TQ, near_tile_weight(NQ, D));
        un.f0 = fp.f0;
        un.fs = fp.fs;
        un.nf = fp.nf;
    }
    un.nn = 0;
    un.wn = un.w;
    auto issue = [&](int u) {  // DMA of unit u into slot u % 2; returns its vector-memory op count
        const int kd = un.kind(u);
        uint8_t* slot = ring + (u & 1) * SLOT;
        if (kd == kFarUnit) {
            if constexpr (TQ) dma_tq<D>(a, bkv, un.tile(u), lane, slot);
            else if constexpr (G32) dma_g32<D>(a, bkv, un.tile(u), lane, slot);
            else dma_far<D>(a, bkv, un.tile(u), lane, slot);
        }
        else if (kd != kNone) dma_near<D, NP>(a, bkv, un.tile(u), kd == kNearV, un.part(u), lane, slot);
        return kd == kNone ? 0 : kd == kFarUnit ? FAR_OPS : NEAR_OPS;
    };
    // ---- the query -> LDS as the B operand of the score MFMA,
    // [qd][s][j][4 halves], by LDS DMA issued before the ring's: the waits
    // below then cover it without waiting for the ring, and no LDS store is
    // needed (the compiler orders LDS stores after every in-flight DMA).
    // Dword w = ((qd * NS + s) * 4 + j) * 2 + e holds dims 4s + 2e, +1 of
    // head 4qd + j; heads past the group read head 0's row (finite values
    // whose results are never written).  TurboQuant stages its own query.
    if constexpr (!TQ) {
        constexpr int QW = NQ * NS * 8;
        static_assert(QW % kWave == 0, "whole-wave query DMA");
        uint8_t* qw = (uint8_t*)(qs + wave * QCOPY);  // this wave's copy (wave-uniform)
#pragma unroll
        for (int k = 0; k < QW / kWave; k++) {
            const int wd = k * kWave + lane, e = wd & 1, jj = (wd >> 1) & 3, s = (wd >> 3) % NS;
            const int h = 4 * ((wd >> 3) / NS) + jj;
            const uint16_t* src = a.q + ((int64_t)b * a.Hq + head0 + (h < ng ? h : 0)) * D + 4 * s + 2 * e;
            __builtin_amdgcn_global_load_lds((const void*)src, (FKV_LDS void*)(qw + k * kWave * 4), 4, 0, 0);
        }
    }
    // the wave's first two far tiles need no device state either.  Behind
    // the launch's first 25 MB of tile requests the query's loads come back
    // late, so the second tile is issued only once the query has landed,
    // and rows of two or more head quads (fp8 far tier), whose tiles are
    // heavier, issue the first one then too (measured: C5 34.5 -> 33.7 us,
    // C3-16K 41.6 -> 41.2 us; rows of one quad lose 0.1-0.2 us when their
    // first tile waits as well)
    constexpr bool QFIRST = !TQ && NQ >= 2;
    if (!TQ && !QFIRST && un.nf > 0) issue(0);
    // TurboQuant: the rotation matrices' slices and the query are loaded
    // together, before any tile: the first far tile's DMA is issued once the
    // rotation is done, so the waits for the rotation's operands (in-order
    // counter) do not also wait for a tile behind 25 MB of others (measured:
    // C4 18.9 -> 18.3 us; issuing both first tiles then is slower, 19.3)
    TqRotation<D> rot;
    constexpr int NT = kWave * WPG;  // threads of the workgroup
    uint16_t tq_q[TQ ? (NQ * NS * 16 + NT - 1) / NT : 1];
    if constexpr (TQ) {
        tq_rotation_load<D, WPG>(a, rot, wave, lane);
        // unconditional loads (heads past the group read head 0 and are
        // zeroed when stored; indices past the arrays wrap)
#pragma unroll
        for (int k = 0; k < (NQ * NS * 16 + NT - 1) / NT; k++) {
            const int i = (threadIdx.x + NT * k) % (NQ * NS * 16);
            const int e = i & 3, jj = (i >> 2) & 3, sq = i >> 4;
            const int s = sq % NS, h = 4 * (sq / NS) + jj;
            tq_q[k] = a.q[((int64_t)b * a.Hq + head0 + (h < ng ? h : 0)) * D + 4 * s + e];
        }
    }
    // the second far tile follows the query wait below (TurboQuant: in the
    // stream; the waits for the rotation operands would also wait for it)
    const bool early1 = !TQ && un.nf > 1;
    // near_valid and a device decode count are written only by earlier
    // launches, so they are read as constant memory (scalar loads, whose
    // counter is not the one the ring's DMA uses)
    const int nv = (int)*(const FKV_CONST uint32_t*)(uintptr_t)(a.blob + a.L.near_valid + 4 * (int64_t)kvh);
    // far keys' score factor: 1/sqrt(D) times the row's fp8 key scale (1
    // unless the handle holds per-head-scaled keys: the scale folds into the
    // score instead of the keys, so the far tile's arithmetic is unchanged)
    const float far_scale = !EXT || TQ || !a.kscale
                                ? a.inv_sqrt_d
                                : a.inv_sqrt_d * *(const FKV_CONST float*)(uintptr_t)(a.kscale + bkv);
    const SpikeTiles spk{SPK ? a.tmax + ((int64_t)b * a.Hq + head0) * a.tmax_stride : nullptr, a.tmax_stride, ng};
    const int nd_raw = a.n_dec_dev ? *(const FKV_CONST int32_t*)(uintptr_t)a.n_dec_dev : a.n_dec;
    float asum[NQ];
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) asum[qd] = 0.f;
    if constexpr (TQ) {
#pragma unroll
        for (int k = 0; k < (NQ * NS * 16 + NT - 1) / NT; k++) {
            const int i = threadIdx.x + NT * k, h = 4 * ((i >> 4) / NS) + ((i >> 2) & 3);
            if (i < NQ * NS * 16) qs[i] = h < ng ? tq_q[k] : (uint16_t)0;
        }
        lds_barrier();
        tq_rotate_query<D, NQ, WPG>(a, rot, QOperand<NS>{qs, j * 4}, qf, qt, rsum, wave, lane);
        if (un.nf > 0) issue(0);
        if (a.tq_alpha != 0.f) {
#pragma unroll
            for (int qd = 0; qd < NQ; qd++) asum[qd] = rsum[4 * qd + j];
        }
    }
    // a decode length kept on the device (graph-captured callers) is clamped
    const int n_dec = a.n_dec_dev ? (nd_raw < 0 ? 0 : nd_raw > a.dec_stride ? a.dec_stride : nd_raw) : nd_raw;
    const int nt_near = (int)cdiv(nv, kTile);
    {
        const int n0 = near_deal_start(TQ, un.N, (int)cdiv(a.L.F, kTile), near_tile_weight(NQ, D), REC);
        un.wn = (un.w - n0 + un.N) % un.N;
    }
    un.nn = un.wn < nt_near ? (int)cdiv(nt_near - un.wn, un.N) : 0;
    if (un.nf == 0) issue(0);

    Lane<D, NQ> st;
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        st.m[qd] = -INFINITY;
        st.lsum[qd] = 0.f;
#pragma unroll
        for (int z = 0; z < D / 32; z++) st.zsum[qd][z] = 0.f;
        st.mn[qd] = INFINITY;
        st.mx[qd] = -INFINITY;
        st.arg[qd] = INT_MAX;
#pragma unroll
        for (int dh = 0; dh < NH; dh++) st.acc[qd][dh] = fkv_f4{0.f, 0.f, 0.f, 0.f};
    }
    // q operand reads from LDS (see QOperand)
    const QOperand<NS> qop{qs + (TQ ? 0 : wave * QCOPY), j * 4};
    const QOperand<NS> qrop{qt, j * 4}, qkop{qt + (TQ ? NQ * NS * 16 : 0), j * 4};
    if constexpr (TQ) {
        lds_barrier();
    } else {
        // the query DMA is this wave's oldest vector-memory op: wait for it
        // but not for the ring (the wave's own copy: no barrier), then issue
        // the second far tile (QFIRST rows: the first two)
        if (QFIRST) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            if (un.nf > 0) issue(0);
            if (early1) issue(1);
        } else if (early1) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(FAR_OPS) : "memory");
            issue(1);
        } else if (un.nf > 0) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(FAR_OPS) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
    }

    // rows of one head quad keep the query operands in registers
    using QSel = std::conditional_t<NQ == 1, QReg<NS>, QOperand<NS>>;
    QSel qx, qrx, qkx;
    if constexpr (NQ == 1) {
        if constexpr (TQ) {
            qrx.load(qrop);
            qkx.load(qkop);
        } else {
            qx.load(qop);
        }
    } else {
        qx = qop;
        qrx = qrop;
        qkx = qkop;
    }

    FKV_STAMP_AT(threadIdx.x == 0, 1);
    // ---- the stream: unit u is computed while unit u + 1 streams in ----
    fkv_f4 sacc[NQ];  // near scores, carried from a K unit to its V unit
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) sacc[qd] = fkv_f4{0.f, 0.f, 0.f, 0.f};
    fkv_h4 w4n[NQ];   // near P.V weights, carried between V parts (NP = 2)
    bool anyn = false;
    const int nu = un.count();
    for (int u = 0; u < nu; u++) {
        // the slot refilled now was read by unit u - 1, whose reads completed
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int pend = (u == 0 && early1) ? FAR_OPS : issue(u + 1);  // unit 1 may be in flight already
        // unit u's loads are complete once at most unit u + 1's are pending
        if (pend == FAR_OPS) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(FAR_OPS) : "memory");
        else if (pend == NEAR_OPS) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NEAR_OPS) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const uint8_t* slot = ring + (u & 1) * SLOT;
        const int kd = un.kind(u), tile = un.tile(u);
        if (kd == kFarUnit) {
            if constexpr (TQ) {
                TqTile<D> r;
                lds_tq(r, slot, lane);
                tq_far_compute<D, NQ>(st, r, tile, lane, a, qrx, qkx, asum);
            } else if constexpr (G32) {
                FarTileG<D> r;
                lds_g32(r, slot, lane);
                g32_far_compute<D, NQ, SPK>(st, r, tile, a.L.F, lane, far_scale, qx, spk);
            } else {
                FarTile<D> r;
                lds_far(r, slot, lane);
                far_compute<D, NQ, SPK>(st, r, tile, a.L.F, blk, far_scale, qx, spk);
            }
        } else if (kd == kNearK) {
            // near tiles: the unrotated query
            if constexpr (TQ) near_scores_lds<D, NQ, NP>(sacc, slot, lane, qop, un.part(u));
            else near_scores_lds<D, NQ>(sacc, slot, lane, qx);
        } else {
            if constexpr (NP == 2) {
                if (un.part(u) == 0) near_pv_lds_part<D, NQ, 0>(st, sacc, w4n, anyn, slot, lane, tile, nv, a.inv_sqrt_d);
                else near_pv_lds_part<D, NQ, 1>(st, sacc, w4n, anyn, slot, lane, tile, nv, a.inv_sqrt_d);
            } else {
                near_pv_lds<D, NQ>(st, sacc, slot, lane, tile, nv, a.inv_sqrt_d);
            }
        }
    }
    // no LDS write may land after the ring is reused or the wave ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- decode buffer (row-major in global memory): tile d to wave
    // dec_wave0 + d mod N (the host picks the least loaded waves).  The far
    // split does not depend on the decode length: a device-held count gives
    // the same partition, and the same bits, as the host count.
    const int nt_dec = (int)cdiv(n_dec, kTile);
    for (int d = (un.w - a.dec_wave0 + un.N) % un.N; d < nt_dec; d += un.N)
    {
        if constexpr (TQ) dec_tile<D, NQ>(st, a, n_dec, bkv, d, lane, qop, ring);
        else dec_tile<D, NQ>(st, a, n_dec, bkv, d, lane, qx, ring);
    }

    FKV_STAMP_AT(lane == 0, 2 + wave);
    // ---- per-head reduction over the 16 lanes (lane % 4 == head) ----
    // Rows of 2..4 splits: every wave publishes its own record (record
    // split * 4 + wave) straight from registers and the last workgroup merges
    // 4 records per split.  Otherwise the 4 waves merge their records in LDS
    // first (one record per split, or the outputs when a row is one split).
    const int row = (int)(bkv * a.head_groups + hgrp);  // (b, kv_head, head group)
    // rows are spaced for the widest row (a last head group may be narrower)
    float* part = a.ws + (int64_t)row * a.num_splits * a.wave_recs * min(a.hpg, a.G) * RS;
    const bool own_rec = a.wave_recs == WPG;
    float* wr = smem + wave * NHW * RS;
    // this wave's record in the workspace (coherent buffer stores, sc1: the
    // cache policy of agent-scope atomic stores)
    const __amdgpu_buffer_rsrc_t wrec = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(part + (int64_t)(split * WPG + wave) * ng * RS), (short)0, ng * RS * 4, 0x00020000);
    if (!own_rec && !SEP_REC) __syncthreads();  // every wave is done with its ring: the records reuse it
#pragma unroll
    for (int qd = 0; qd < NQ; qd++) {
        const float l = head_sum<true>(st.lsum[qd]), mn = head_min(st.mn[qd]);
        float mx = st.mx[qd];
        int arg = st.arg[qd];
        head_argmax(mx, arg);
        // INT4 correction of head j (per 64-dim half dh): minus the +16
        // decode offset and the 7.5 centring, plus the zero points.
        // Group-32 V: the lane's dims are group 2dh + half; its own half's
        // tokens reduce over the 16 lanes of the head in this half, the
        // other half's tokens come across from the other half's lanes.
        float corr[NH];
        if constexpr (G32) {
            const int half = lane >> 5;
#pragma unroll
            for (int dh = 0; dh < NH; dh++) {
                const float zo = head_sum<false>(st.zsum[qd][dh]);
                const float zx = head_sum<false>(st.zsum[qd][NH + dh]);
                corr[dh] = zo + swap_halves(zx, half);
            }
        } else {
            const float z = head_sum<true>(st.zsum[qd][0]);
#pragma unroll
            for (int dh = 0; dh < NH; dh++) corr[dh] = z;
        }
        const int h = 4 * qd + j;
        const float hdr[5] = {st.m[qd], l, mn, mx, __int_as_float(arg)};
        if (own_rec) {
            if (lane < 4 && h < ng) {
                const fkv_v4u hv = __builtin_bit_cast(fkv_v4u, fkv_f4{hdr[0], hdr[1], hdr[2], hdr[3]});
                // header words 4, 5: the argmax and this workgroup's XCD
                const fkv_v2u ax = fkv_v2u{(uint32_t)arg, xcc_id()};
                if (xcd_local) {
                    __builtin_amdgcn_raw_buffer_store_b128(hv, wrec, h * RS * 4, 0, kCpolSc0);
                    __builtin_amdgcn_raw_buffer_store_b64(ax, wrec, h * RS * 4 + 16, 0, kCpolSc0);
                } else {
                    __builtin_amdgcn_raw_buffer_store_b128(hv, wrec, h * RS * 4, 0, kCpolSc1);
                    __builtin_amdgcn_raw_buffer_store_b64(ax, wrec, h * RS * 4 + 16, 0, kCpolSc1);
                }
            }
        } else if (lane < 4 && h < ng) {
#pragma unroll
            for (int e = 0; e < 5; e++) wr[h * RS + e] = hdr[e];
        }
#pragma unroll
        for (int dh = 0; dh < NH; dh++) {
            const float zz[4] = {quad_bcast<0>(corr[dh]), quad_bcast<1>(corr[dh]), quad_bcast<2>(corr[dh]),
                                 quad_bcast<3>(corr[dh])};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (4 * qd + i < ng) {
                    const int e = (4 * qd + i) * RS + kHdr + 64 * dh + lane;
                    const float v = st.acc[qd][dh][i] + zz[i];
                    if (own_rec) {
                        if (xcd_local) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), wrec, e * 4, 0, kCpolSc0);
                        else __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), wrec, e * 4, 0, kCpolSc1);
                    } else {
                        wr[e] = v;
                    }
                }
            }
        }
    }
    if (own_rec) {
        if (a.arrive == nullptr) return;  // merged by merge_kernel (kernel boundary orders it)
        // the arrival is counted once this workgroup's stores are complete
        // (the ordering argument of the merged-record path below)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        FKV_STAMP_AT(threadIdx.x == 0, 20);
        if (threadIdx.x == 0) s_last = arrive_last(a, row, xcd_local);
        __syncthreads();
        FKV_STAMP_AT(threadIdx.x == 0, 21);
        if (!s_last) return;
        merge_finalize_direct<D, WPG, EXT>(a, part, a.num_splits * WPG, ng, b, head0, xcd_local, row);
        if (threadIdx.x == 0) rearm(a, row, xcd_local);
#ifdef FKV_PHASE_STAMPS
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
#endif
        FKV_STAMP_AT(threadIdx.x == 0, 22);
        return;
    }
    __syncthreads();

    // ---- merge the waves' records into wave 0's ----
    // Wave w merges heads w, w + WPG, ...: every record value of its heads
    // is read into registers before the first merged value is written (the
    // writes go to wave 0's records, which the same loads read), so the
    // reads issue as one batch.
    {
        constexpr int HPW = (NHW + WPG - 1) / WPG;  // heads per wave, at most
        constexpr int VD = D / kWave;               // values per lane and head
        float hm[HPW][WPG], hl[HPW][WPG], hn[HPW][WPG], hx[HPW][WPG];
        int ha[HPW][WPG];
        float hv[HPW][WPG][VD];
#pragma unroll
        for (int i = 0; i < HPW; i++) {
            const int h = wave + i * WPG;
            if (h < ng) {
#pragma unroll
                for (int w = 0; w < WPG; w++) {
                    const float* r = smem + w * NHW * RS + h * RS;
                    hm[i][w] = r[0];
                    hl[i][w] = r[1];
                    hn[i][w] = r[2];
                    hx[i][w] = r[3];
                    ha[i][w] = __float_as_int(r[4]);
#pragma unroll
                    for (int k = 0; k < VD; k++) hv[i][w][k] = r[kHdr + lane + k * kWave];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < HPW; i++) {
            const int h = wave + i * WPG;
            if (h >= ng) continue;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < WPG; w++) M = fmaxf(M, hm[i][w]);
            float sc[WPG];
            float L = 0.f, mn2 = INFINITY, mx2 = -INFINITY;
            int arg2 = INT_MAX;
#pragma unroll
            for (int w = 0; w < WPG; w++) {
                sc[w] = hm[i][w] == -INFINITY ? 0.f : __expf(hm[i][w] - M);
                L += sc[w] * hl[i][w];
                mn2 = fminf(mn2, hn[i][w]);
                pick_max(mx2, arg2, hx[i][w], ha[i][w]);
            }
#pragma unroll
            for (int k = 0; k < VD; k++) {
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < WPG; w++) v += sc[w] * hv[i][w][k];
                smem[h * RS + kHdr + lane + k * kWave] = v;
            }
            if (lane == 0) {
                smem[h * RS + 0] = M;
                smem[h * RS + 1] = L;
                smem[h * RS + 2] = mn2;
                smem[h * RS + 3] = mx2;
                smem[h * RS + 4] = __int_as_float(arg2);
                smem[h * RS + 5] = __uint_as_float(xcc_id());  // the writer's XCD (merge check)
            }
        }
    }
    __syncthreads();

    if (a.num_splits == 1) {
        finalize_rows<D, EXT>(a, smem, b, head0, ng);
        return;
    }
    // ---- split-K: publish this split's record ----
    if (a.arrive == nullptr) {  // merged by merge_kernel (kernel boundary orders it)
        for (int i = threadIdx.x; i < ng * RS; i += blockDim.x) part[(int64_t)split * ng * RS + i] = smem[i];
        return;
    }
    // The last split to arrive merges all records (no second launch) and
    // re-arms the counter.  Cross-workgroup ordering without cache-wide
    // maintenance: the records are written with agent-scope atomic stores
    // (coherent across XCDs, nothing left dirty in a non-coherent L2), each
    // thread waits for its stores to complete before the barrier, then one
    // agent-scope RMW counts the arrival; the last workgroup reads the
    // records back with agent-scope atomic loads.  (A release/acquire fence
    // pair would write back and invalidate the whole L2 per workgroup.)
    // XCD-local: the row's splits share one L2, so plain stores, an L2
    // atomic and sc0 loads order the same way without waiting for memory.
    float* rec = part + (int64_t)split * ng * RS;
    if (xcd_local) {
        for (int i = threadIdx.x; i < ng * RS; i += blockDim.x)
            __hip_atomic_store(rec + i, smem[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
        for (int i = threadIdx.x; i < ng * RS; i += blockDim.x)
            __hip_atomic_store(rec + i, smem[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    FKV_STAMP_AT(threadIdx.x == 0, 20);
    if (threadIdx.x == 0) s_last = arrive_last(a, row, xcd_local);
    __syncthreads();
    FKV_STAMP_AT(threadIdx.x == 0, 21);
    if (!s_last) return;
    // every record (this split's included) is in global memory (the row's
    // L2) now
    merge_finalize_direct<D, WPG, EXT>(a, part, a.num_splits, ng, b, head0, xcd_local, row);
    if (threadIdx.x == 0) rearm(a, row, xcd_local);
#ifdef FKV_PHASE_STAMPS
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#endif
    FKV_STAMP_AT(threadIdx.x == 0, 22);
}

typedef void (*AttnKernel)(AttnArgs);

// The fp8 and group-32 attention kernels (fmt 0, 2) of rows of one head
// quad (fkv_attn_q1.hip; EXT: fkv_attn_q1x.hip) and of nq = 2..4 quads
// (fkv_attn_qn.hip, fkv_attn_qnx.hip); spk picks the top-K kernels.
AttnKernel attn_kernel_one_quad(int D, int fmt, bool ext, bool spk);
AttnKernel attn_kernel_quads(int D, int fmt, int nq, bool ext, bool spk);

}  // namespace fkv
