/*
 * fkv_oracle.c -- CPU restatement of the reference FoveatedKV decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path (foveated_kv_amd/)
 * may link, load or call this file.  It is the checker that tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * library against, and it is never the thing measured as the product.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the samfurr/foveated_kv repository root).  The arithmetic is written
 * from the reference's semantics, not copied: fp16 values are handled as
 * raw uint16 bit patterns and converted with the exact routines below.
 *
 * Pinning status of each function (how each is checked in tests/):
 *   orc_fp16_to_e4m3        pinned: exhaustive 65536-pattern value-semantics
 *                           check + torch float8_e4m3fn RNE on the normal range
 *   orc_fp16_to_e4m3_py     pinned: exhaustive divergence count vs the Metal
 *                           encoder (18,688 patterns) + value-semantics check
 *   orc_e4m3_to_fp16        pinned: closed form + torch float8_e4m3fn decode
 *   orc_quant_int4_*        pinned: invariants, crafted .5 ties, legacy fixture
 *                           nibble order
 *   orc_tier_boundaries     pinned: known answers (S=1000 -> 100/900, config
 *                           table of the hot-path scope)
 *   orc_split_plan          pinned: known answers for configs 1-3
 *   orc_attend_kernel       pinned: 6 legacy fixtures, fp64 brute force,
 *                           split-count invariance, spike_case fixture
 *   orc_attend_formulation  pinned: 6 legacy fixtures, brute force
 *   orc_attend_turbo        pinned: far scores against the dequantised-key
 *                           identities (exact reconstruction -> q.k_hat; QJL
 *                           term = sqrt(pi/2) x the formulation's q.r_hat),
 *                           fp64 brute force, split-count invariance
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* IEEE binary16 / bfloat16 conversions (exact, round-to-nearest-even)      */
/* ------------------------------------------------------------------------ */

ORC_API float orc_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    int32_t e = (h >> 10) & 0x1f;
    uint32_t m = h & 0x3ffu;
    float v;
    if (e == 0) {
        v = ldexpf((float)m, -24); /* subnormal: m * 2^-24 (exact in fp32) */
    } else if (e == 31) {
        v = m ? NAN : INFINITY;
    } else {
        v = ldexpf((float)(m | 0x400u), e - 25);
    }
    return sign ? -v : v;
}

/* Round a double to the nearest binary16 (ties to even).  Used for every
 * fp16 store the reference performs ((half)x casts, astype(float16)). */
ORC_API uint16_t orc_d2h(double x) {
    uint16_t sign = signbit(x) ? 0x8000u : 0u;
    double a = fabs(x);
    if (isnan(x)) return (uint16_t)(sign | 0x7e00u);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (a < ldexp(1.0, -14)) {
        /* subnormal range: quantum 2^-24 */
        double q = a * 16777216.0; /* a / 2^-24 */
        double r = nearbyint(q);   /* default rounding mode: ties-to-even */
        return (uint16_t)(sign | (uint16_t)r); /* r <= 1024 -> may become min normal */
    }
    int e;
    double f = frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) */
    /* binary16 significand has 11 bits: quantum 2^(e-11) */
    double q = ldexp(a, 11 - e);
    double r = nearbyint(q); /* in [1024, 2048] */
    (void)f;
    if (r >= 2048.0) { r = 1024.0; e += 1; }
    int exp16 = e - 1 + 15;
    if (exp16 >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)(exp16 << 10) | ((uint16_t)r & 0x3ffu));
}

ORC_API uint16_t orc_f2h(float x) { return orc_d2h((double)x); }

ORC_API float orc_bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

ORC_API uint16_t orc_f2bf(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

/* ------------------------------------------------------------------------ */
/* fp8 E4M3 encode / decode                                                  */
/* ------------------------------------------------------------------------ */

/* Metal encoder: csrc/kernels/foveated_compress.metal:39-66.
 * Saturation and underflow are decided on the re-biased exponent BEFORE
 * rounding; a rounding carry that reaches exponent 15 saturates to 0x7E. */
ORC_API uint8_t orc_fp16_to_e4m3(uint16_t bits) {
    uint32_t sign = bits >> 15;
    int exp16 = (bits >> 10) & 0x1f;
    uint32_t mant = bits & 0x3ffu;
    if (exp16 == 0) return (uint8_t)(sign << 7);
    if (exp16 == 31) return (uint8_t)((sign << 7) | 0x7eu);
    int e8 = exp16 - 8;
    if (e8 >= 15) return (uint8_t)((sign << 7) | 0x7eu);
    if (e8 <= 0) return (uint8_t)(sign << 7);
    uint32_t keep = mant >> 7;           /* top 3 mantissa bits            */
    uint32_t half_bit = (mant >> 6) & 1u; /* first dropped bit             */
    uint32_t rest = (mant & 0x3fu) != 0;  /* any lower dropped bit         */
    if (half_bit && (rest || (keep & 1u))) {
        keep += 1;
        if (keep == 8) { keep = 0; e8 += 1; }
        if (e8 >= 15) return (uint8_t)((sign << 7) | 0x7eu);
    }
    return (uint8_t)((sign << 7) | ((uint32_t)e8 << 3) | keep);
}

/* Python encoder: src/foveated_kv/mlx_foveated.py:528-566.  Rounds first,
 * then tests underflow on the carried exponent and clamps overflow to 0x76. */
ORC_API uint8_t orc_fp16_to_e4m3_py(uint16_t bits) {
    int32_t b = bits;
    int32_t sign = (b >> 15) & 1;
    int32_t exp16 = (b >> 10) & 0x1f;
    int32_t mant = b & 0x3ff;
    int32_t exp8 = exp16 - 8;
    int32_t keep = mant >> 7;
    int32_t half_bit = (mant >> 6) & 1;
    int32_t rest = (mant & 0x3f) != 0;
    int32_t up = half_bit & (rest | (keep & 1));
    int32_t m3 = keep + up;
    int32_t carry = m3 >= 8;
    if (carry) m3 = 0;
    exp8 += carry;
    int under = (exp8 <= 0) || (exp16 == 0);
    int over = (exp8 >= 15) || (exp16 == 31);
    if (under) { exp8 = 0; m3 = 0; }
    if (over) { exp8 = 14; m3 = 6; }
    return (uint8_t)(((sign << 7) | (exp8 << 3) | m3) & 0xff);
}

/* Decode LUT: csrc/kernels/foveated_attn.metal:237-253 (and the Python
 * twin mlx_foveated.py:76-91).  Exponent 0 decodes to signed zero whatever
 * the mantissa; every other code maps to fp16 by re-biasing the exponent. */
ORC_API uint16_t orc_e4m3_to_fp16(uint8_t v) {
    uint32_t sign = v >> 7, e = (v >> 3) & 0xfu, m = v & 7u;
    if (e == 0) return (uint16_t)(sign << 15);
    return (uint16_t)((sign << 15) | ((e + 8) << 10) | (m << 7));
}

ORC_API void orc_encode_fp8(const uint16_t* src, uint8_t* dst, int64_t n, int python_semantics) {
    for (int64_t i = 0; i < n; i++)
        dst[i] = python_semantics ? orc_fp16_to_e4m3_py(src[i]) : orc_fp16_to_e4m3(src[i]);
}

/* ------------------------------------------------------------------------ */
/* INT4 per-token quantisation                                               */
/* ------------------------------------------------------------------------ */

/* Metal: csrc/kernels/foveated_compress.metal:153-205.
 * rows of D fp16 -> packed (D/2 bytes, even dim in the low nibble), fp16
 * scale = half(max((max-min)/15, 1e-8)), fp16 zero = half(min).  Codes use
 * the fp32 scale and Metal round() = half away from zero. */
ORC_API void orc_quant_int4_rows(const uint16_t* src, int64_t rows, int D,
                                 uint8_t* packed, uint16_t* scale, uint16_t* zero) {
    for (int64_t r = 0; r < rows; r++) {
        const uint16_t* x = src + r * D;
        float mn = INFINITY, mx = -INFINITY;
        for (int d = 0; d < D; d++) {
            float v = orc_h2f(x[d]);
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
        float sc = fmaxf((mx - mn) / 15.0f, 1e-8f);
        scale[r] = orc_f2h(sc);
        zero[r] = orc_f2h(mn);
        for (int p = 0; p < D / 2; p++) {
            float lo = roundf((orc_h2f(x[2 * p]) - mn) / sc);
            float hi = roundf((orc_h2f(x[2 * p + 1]) - mn) / sc);
            lo = fminf(fmaxf(lo, 0.0f), 15.0f);
            hi = fminf(fmaxf(hi, 0.0f), 15.0f);
            packed[r * (D / 2) + p] = (uint8_t)((uint32_t)lo | ((uint32_t)hi << 4));
        }
    }
}

/* Python: src/foveated_kv/mlx_foveated.py:569-600.  scale==0 -> 1 and
 * mx.round (ties to even). */
ORC_API void orc_quant_int4_rows_py(const uint16_t* src, int64_t rows, int D,
                                    uint8_t* packed, uint16_t* scale, uint16_t* zero) {
    for (int64_t r = 0; r < rows; r++) {
        const uint16_t* x = src + r * D;
        float mn = INFINITY, mx = -INFINITY;
        for (int d = 0; d < D; d++) {
            float v = orc_h2f(x[d]);
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
        float sc = (mx - mn) / 15.0f;
        if (sc == 0.0f) sc = 1.0f;
        scale[r] = orc_f2h(sc);
        zero[r] = orc_f2h(mn);
        for (int p = 0; p < D / 2; p++) {
            float lo = rintf((orc_h2f(x[2 * p]) - mn) / sc);
            float hi = rintf((orc_h2f(x[2 * p + 1]) - mn) / sc);
            lo = fminf(fmaxf(lo, 0.0f), 15.0f);
            hi = fminf(fmaxf(hi, 0.0f), 15.0f);
            packed[r * (D / 2) + p] = (uint8_t)((uint32_t)lo | ((uint32_t)hi << 4));
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Tier boundaries and split plan                                            */
/* ------------------------------------------------------------------------ */

/* src/foveated_kv/mlx_foveated.py:128-169 (C++ twin foveated_compress.cpp:107-126).
 * out[] = { n_sinks, window, near_from_mid, far_count, R_actual,
 *           N_near_padded, mid_start, mid_end, near_mid_start, headroom } */
ORC_API void orc_tier_boundaries(double near_pct, int n_sinks_cfg, int window_cfg,
                                 double headroom_pct, int headroom_min, int S, int* out) {
    int n_sinks = n_sinks_cfg < S ? n_sinks_cfg : S;
    int rest = S - n_sinks > 0 ? S - n_sinks : 0;
    int window = window_cfg < rest ? window_cfg : rest;
    int reserved = n_sinks + window;
    int r_total = (int)((double)S * near_pct); /* Python int(): truncation */
    if (r_total < reserved) r_total = reserved;
    int far_count = S - r_total;
    if (far_count < 0) { far_count = 0; r_total = S; }
    int mid_start = n_sinks;
    int mid_end = window > 0 ? S - window : S;
    int mid_len = mid_end - mid_start > 0 ? mid_end - mid_start : 0;
    int from_mid = r_total - reserved > 0 ? r_total - reserved : 0;
    if (from_mid > mid_len) from_mid = mid_len;
    int r_actual = n_sinks + from_mid + window;
    int headroom = (int)((double)r_actual * headroom_pct);
    if (headroom < headroom_min) headroom = headroom_min;
    int near_mid_start = mid_end - from_mid;
    out[0] = n_sinks;
    out[1] = window;
    out[2] = from_mid;
    out[3] = near_mid_start - mid_start;
    out[4] = r_actual;
    out[5] = r_actual + headroom;
    out[6] = mid_start;
    out[7] = mid_end;
    out[8] = near_mid_start;
    out[9] = headroom;
}

/* csrc/foveated_attn.cpp:26-38 and :178-181: out = {split_size, num_splits, max_splits} */
ORC_API void orc_split_plan(int s_total, int* out) {
    const int base = 256, cap = 16;
    int split = base;
    if (s_total > base * cap) split = ((s_total + cap - 1) / cap + 255) / 256 * 256;
    int n = (s_total + split - 1) / split;
    int mx = n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : n <= 8 ? 8 : 16;
    out[0] = split;
    out[1] = n;
    out[2] = mx;
}

/* ------------------------------------------------------------------------ */
/* Fused two-tier attention: kernel semantics                                */
/* ------------------------------------------------------------------------ */

typedef struct {
    double m, l;
    double* acc; /* D */
    double min_near, max_far;
    int far_tok;
} orc_state;

static void orc_accum(orc_state* st, double s, const double* v, int D) {
    /* softmax_accum: csrc/kernels/foveated_attn.metal:75-87 */
    double m_new = st->m > s ? st->m : s;
    double alpha = exp(st->m - m_new);
    double w = exp(s - m_new);
    st->l = alpha * st->l + w;
    for (int d = 0; d < D; d++) st->acc[d] = alpha * st->acc[d] + w * v[d];
    st->m = m_new;
}

/* foveated_2tier: csrc/kernels/foveated_attn.metal:181-432 with the split
 * plan of csrc/foveated_attn.cpp:164-240.  Computed in fp64 from the
 * kernel's fp32 inputs (q pre-scaled by rsqrt(D) in fp32, :258-261; far V
 * dequantised as fma(nibble, scale, zero) without fp16 rounding, :152-174).
 *
 *   q        (B,Hq,D)        fp16 bits
 *   near_k/v (B,Hkv,Npad,D)  fp16 bits
 *   near_valid (Hkv)          per-KV-head valid count, shared across batch (:289)
 *   far_k    (B,Hkv,F,D)     E4M3 codes
 *   far_k_f16 (B,Hkv,F,D)    optional fp16 far keys used instead of the LUT
 *                            decode of far_k (lets the legacy INT8-K fixtures
 *                            drive the INT4-V far path); NULL for fp8 keys
 *   far_v    (B,Hkv,F,D/2)   INT4 packed, low nibble = even dim
 *   far_vs/vz (B,Hkv,F)      fp16 bits (v_group 0: one scale / zero per
 *                            token, the reference); (B,Hkv,F,D/v_group) with
 *                            v_group > 0: one per v_group dims (the group-32
 *                            extension: the reference's per-token arithmetic
 *                            applied to each group)
 *   dec_k/v  (B,Hkv,n_dec,D) fp16 bits
 *   far_k_scale (B,Hkv) fp32 or NULL: per-head fp8 key scale (the
 *                            benchmark's "per-head-scaled fp8 E4M3" keys, an
 *                            extension: the reference's keys are unscaled);
 *                            a far key is decode(code) * scale
 *   split_size/num_splits <= 0 -> reference adaptive plan
 *   gate != 0 -> skip V of far tokens with s < m - 16 (:311-360)
 *   out (B,Hq,D) fp64; flags/tokens (B,Hq); max_far/min_near (B,Hq) optional;
 *   far_scores (B,Hq,F) fp64 optional: every far token's score (the input
 *   of the top-K spike selection, oracle/__init__.py spike_topk)
 */
ORC_API int orc_attend_kernel(int B, int Hq, int Hkv, int D, int Npad, int F, int n_dec,
                              const uint16_t* q, const uint16_t* near_k, const uint16_t* near_v,
                              const uint32_t* near_valid, const uint8_t* far_k,
                              const uint16_t* far_k_f16,
                              const uint8_t* far_v, const uint16_t* far_vs,
                              const uint16_t* far_vz, const uint16_t* dec_k,
                              const uint16_t* dec_v, const float* far_k_scale, float spike_margin,
                              int split_size, int num_splits, int gate, int v_group, double* out,
                              int32_t* flags, int32_t* tokens, double* max_far_out, double* min_near_out,
                              double* far_scores_out) {
    if (Hkv <= 0 || Hq % Hkv != 0 || D <= 0) return -1;
    if (v_group < 0 || (v_group > 0 && D % v_group != 0)) return -1;
    const int G = Hq / Hkv;
    const int NGV = v_group > 0 ? D / v_group : 1; /* scale / zero entries per far token */
    const int s_total = Npad + F + n_dec;
    if (split_size <= 0 || num_splits <= 0) {
        int plan[3];
        orc_split_plan(s_total, plan);
        split_size = plan[0];
        num_splits = plan[1];
    }
    const float inv_sqrt_d = 1.0f / sqrtf((float)D);
    double* qreg = (double*)malloc(sizeof(double) * D);
    double* vv = (double*)malloc(sizeof(double) * D);
    double* racc = (double*)malloc(sizeof(double) * D);
    orc_state* sp = (orc_state*)malloc(sizeof(orc_state) * num_splits);
    double* accbuf = (double*)malloc(sizeof(double) * D * num_splits);
    if (!qreg || !vv || !racc || !sp || !accbuf) return -2;

    for (int b = 0; b < B; b++) {
        for (int hq = 0; hq < Hq; hq++) {
            const int kvh = hq / G;
            const int64_t bkv = (int64_t)b * Hkv + kvh;
            for (int d = 0; d < D; d++) {
                float qf = orc_h2f(q[((int64_t)b * Hq + hq) * D + d]) * inv_sqrt_d;
                qreg[d] = (double)qf;
            }
            for (int s = 0; s < num_splits; s++) {
                orc_state* st = &sp[s];
                st->m = -INFINITY;
                st->l = 0.0;
                st->acc = accbuf + (int64_t)s * D;
                for (int d = 0; d < D; d++) st->acc[d] = 0.0;
                st->min_near = INFINITY;
                st->max_far = -INFINITY;
                st->far_tok = -1;
                int g0 = s * split_size;
                int g1 = g0 + split_size < s_total ? g0 + split_size : s_total;
                int near0 = g0 < Npad ? g0 : Npad;
                int near1 = g1 < Npad ? g1 : Npad;
                int far0 = g0 > Npad ? (g0 - Npad < F ? g0 - Npad : F) : 0;
                int far1 = g1 > Npad ? (g1 - Npad < F ? g1 - Npad : F) : 0;
                int nf = Npad + F;
                int dec0 = g0 > nf ? (g0 - nf < n_dec ? g0 - nf : n_dec) : 0;
                int dec1 = g1 > nf ? (g1 - nf < n_dec ? g1 - nf : n_dec) : 0;
                int nv = (int)near_valid[kvh];
                int near_end = near1 < nv ? near1 : nv;
                for (int t = near0; t < near_end; t++) {
                    const uint16_t* kr = near_k + (bkv * Npad + t) * D;
                    const uint16_t* vr = near_v + (bkv * Npad + t) * D;
                    double sc = 0.0;
                    for (int d = 0; d < D; d++) sc += qreg[d] * (double)orc_h2f(kr[d]);
                    if (sc < st->min_near) st->min_near = sc;
                    for (int d = 0; d < D; d++) vv[d] = orc_h2f(vr[d]);
                    orc_accum(st, sc, vv, D);
                }
                const double ks = far_k_scale ? (double)far_k_scale[bkv] : 1.0;
                for (int t = far0; t < far1; t++) {
                    double sc = 0.0;
                    if (far_k_f16) {
                        const uint16_t* kr = far_k_f16 + (bkv * F + t) * D;
                        for (int d = 0; d < D; d++) sc += qreg[d] * (double)orc_h2f(kr[d]);
                    } else {
                        const uint8_t* kr = far_k + (bkv * F + t) * D;
                        for (int d = 0; d < D; d++)
                            sc += qreg[d] * (double)orc_h2f(orc_e4m3_to_fp16(kr[d]));
                    }
                    sc *= ks;
                    if (far_scores_out) far_scores_out[((int64_t)b * Hq + hq) * F + t] = sc;
                    if (sc > st->max_far) { st->max_far = sc; st->far_tok = t; }
                    if (gate && sc < st->m - 16.0) continue;
                    const uint8_t* vr = far_v + (bkv * F + t) * (D / 2);
                    for (int d = 0; d < D; d++) {
                        const int64_t si = (bkv * F + t) * NGV + (v_group > 0 ? d / v_group : 0);
                        const double vs = orc_h2f(far_vs[si]), vz = orc_h2f(far_vz[si]);
                        const int nib = (d & 1) ? (vr[d >> 1] >> 4) : (vr[d >> 1] & 15);
                        vv[d] = (double)nib * vs + vz;
                    }
                    orc_accum(st, sc, vv, D);
                }
                for (int t = dec0; t < dec1; t++) {
                    const uint16_t* kr = dec_k + (bkv * n_dec + t) * D;
                    const uint16_t* vr = dec_v + (bkv * n_dec + t) * D;
                    double sc = 0.0;
                    for (int d = 0; d < D; d++) sc += qreg[d] * (double)orc_h2f(kr[d]);
                    if (sc < st->min_near) st->min_near = sc;
                    for (int d = 0; d < D; d++) vv[d] = orc_h2f(vr[d]);
                    orc_accum(st, sc, vv, D);
                }
            }
            /* split merge: csrc/kernels/foveated_attn.metal:394-431 */
            double mg = -INFINITY, lg = 0.0, min_near = INFINITY, max_far = -INFINITY;
            int far_tok = -1;
            for (int d = 0; d < D; d++) racc[d] = 0.0;
            for (int s = 0; s < num_splits; s++) {
                orc_state* st = &sp[s];
                if (st->m == -INFINITY) continue;
                double mn = mg > st->m ? mg : st->m;
                double ag = mg > -INFINITY ? exp(mg - mn) : 0.0;
                double as = exp(st->m - mn);
                lg = ag * lg + as * st->l;
                for (int d = 0; d < D; d++) racc[d] = ag * racc[d] + as * st->acc[d];
                mg = mn;
                if (st->min_near < min_near) min_near = st->min_near;
                if (st->max_far > max_far) { max_far = st->max_far; far_tok = st->far_tok; }
            }
            /* note: the reference also skips the spike fields of splits whose
             * m is -inf; such splits saw no token so their fields are neutral */
            double inv_l = lg > 0.0 ? 1.0 / lg : 0.0;
            const int64_t o = ((int64_t)b * Hq + hq);
            for (int d = 0; d < D; d++) out[o * D + d] = racc[d] * inv_l;
            flags[o] = (max_far > min_near + (double)spike_margin) ? 1 : 0;
            tokens[o] = far_tok;
            if (max_far_out) max_far_out[o] = max_far;
            if (min_near_out) min_near_out[o] = min_near;
        }
    }
    free(qreg);
    free(vv);
    free(racc);
    free(sp);
    free(accbuf);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Reference formulation (Python fallback attend)                            */
/* ------------------------------------------------------------------------ */

/* MLXFoveatedLayer.attend: src/foveated_kv/mlx_foveated.py:239-278.
 *   far K   = LUT decode (exact in fp16)                       :76-91
 *   far V   = half(half(nibble * scale) + zero)  (fp16 ops)    :94-108
 *   far_k_scale (B,Hkv) fp32 or NULL: per-head key scale (extension, see
 *             orc_attend_kernel): far K = decode(code) * scale in fp32
 *   keys    = near[:, :, :max(near_valid)] ++ decode ++ far    :256-260, :430-449
 *   q_dtype = 1 (bf16): K/V rounded to bf16 before SDPA        :262-266
 *   SDPA with scale 1/sqrt(D), GQA by repeat                   :268-278
 * Softmax is evaluated in fp64 (MLX SDPA's internal precision is not
 * reproducible here; see the test tolerances).  OpenMP over (b, q_head). */
ORC_API int orc_attend_formulation(int B, int Hq, int Hkv, int D, int Npad, int F, int n_dec,
                                   const uint16_t* q, int q_dtype, const uint16_t* near_k,
                                   const uint16_t* near_v, const uint32_t* near_valid,
                                   const uint8_t* far_k, const uint8_t* far_v,
                                   const uint16_t* far_vs, const uint16_t* far_vz,
                                   const uint16_t* dec_k, const uint16_t* dec_v, int v_group,
                                   const float* far_k_scale, double* out) {
    if (Hkv <= 0 || Hq % Hkv != 0) return -1;
    if (v_group < 0 || (v_group > 0 && D % v_group != 0)) return -1;
    const int NGV = v_group > 0 ? D / v_group : 1;
    const int G = Hq / Hkv;
    int nv_max = 0;
    for (int h = 0; h < Hkv; h++)
        if ((int)near_valid[h] > nv_max) nv_max = (int)near_valid[h];
    if (nv_max > Npad) nv_max = Npad;
    const int T = nv_max + n_dec + F;
    const double scale = 1.0 / sqrt((double)D);
    int err = 0;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; b++) {
        for (int hq = 0; hq < Hq; hq++) {
            double* sc = (double*)malloc(sizeof(double) * (T > 0 ? T : 1));
            double* acc = (double*)malloc(sizeof(double) * D);
            double* qv = (double*)malloc(sizeof(double) * D);
            float* krow = (float*)malloc(sizeof(float) * D);
            if (!sc || !acc || !qv || !krow) {
                err = -2;
                free(sc); free(acc); free(qv); free(krow);
                continue;
            }
            const int kvh = hq / G;
            const int64_t bkv = (int64_t)b * Hkv + kvh;
            const int64_t o = (int64_t)b * Hq + hq;
            for (int d = 0; d < D; d++)
                qv[d] = q_dtype ? orc_bf2f(q[o * D + d]) : orc_h2f(q[o * D + d]);
            /* pass 1: scores */
            double mx = -INFINITY;
            for (int t = 0; t < T; t++) {
                for (int d = 0; d < D; d++) {
                    float kf;
                    if (t < nv_max) kf = orc_h2f(near_k[(bkv * Npad + t) * D + d]);
                    else if (t < nv_max + n_dec)
                        kf = orc_h2f(dec_k[(bkv * n_dec + (t - nv_max)) * D + d]);
                    else if (far_k_scale)
                        kf = orc_h2f(orc_e4m3_to_fp16(far_k[(bkv * F + (t - nv_max - n_dec)) * D + d])) *
                             far_k_scale[bkv];
                    else
                        kf = orc_h2f(orc_e4m3_to_fp16(far_k[(bkv * F + (t - nv_max - n_dec)) * D + d]));
                    krow[d] = q_dtype ? orc_bf2f(orc_f2bf(kf)) : kf;
                }
                double s = 0.0;
                for (int d = 0; d < D; d++) s += qv[d] * (double)krow[d];
                sc[t] = s * scale;
                if (sc[t] > mx) mx = sc[t];
            }
            double l = 0.0;
            for (int d = 0; d < D; d++) acc[d] = 0.0;
            for (int t = 0; t < T; t++) {
                double w = exp(sc[t] - mx);
                l += w;
                for (int d = 0; d < D; d++) {
                    float vf;
                    if (t < nv_max) vf = orc_h2f(near_v[(bkv * Npad + t) * D + d]);
                    else if (t < nv_max + n_dec)
                        vf = orc_h2f(dec_v[(bkv * n_dec + (t - nv_max)) * D + d]);
                    else {
                        int64_t tf = bkv * F + (t - nv_max - n_dec);
                        uint8_t byte = far_v[tf * (D / 2) + d / 2];
                        float nib = (float)((d & 1) ? (byte >> 4) : (byte & 15));
                        const int64_t si = tf * NGV + (v_group > 0 ? d / v_group : 0);
                        float s16 = orc_h2f(far_vs[si]);
                        float z16 = orc_h2f(far_vz[si]);
                        float prod = orc_h2f(orc_f2h(nib * s16));
                        vf = orc_h2f(orc_f2h(prod + z16));
                    }
                    if (q_dtype) vf = orc_bf2f(orc_f2bf(vf));
                    acc[d] += w * (double)vf;
                }
            }
            for (int d = 0; d < D; d++) out[o * D + d] = l > 0.0 ? acc[d] / l : 0.0;
            free(sc); free(acc); free(qv); free(krow);
        }
    }
    return err;
}

/* ------------------------------------------------------------------------ */
/* Near-tier gather (compress_foveal)                                        */
/* ------------------------------------------------------------------------ */

/* csrc/kernels/foveated_compress.metal:76-109 with the parameters of
 * csrc/foveated_compress.cpp:135-143.  src (BH,S,D) -> dst (BH,Npad,D),
 * rows >= R_actual zero. */
ORC_API void orc_compress_foveal(const uint16_t* src, uint16_t* dst, int BH, int S, int D,
                                 int n_sinks, int mid_start, int mid_count, int window_start,
                                 int r_actual, int npad) {
    for (int bh = 0; bh < BH; bh++) {
        for (int t = 0; t < npad; t++) {
            int srct = -1;
            if (t < n_sinks) srct = t;
            else if (t < n_sinks + mid_count) srct = mid_start + (t - n_sinks);
            else if (t < r_actual) srct = window_start + (t - n_sinks - mid_count);
            uint16_t* o = dst + ((int64_t)bh * npad + t) * D;
            if (srct < 0) memset(o, 0, sizeof(uint16_t) * D);
            else memcpy(o, src + ((int64_t)bh * S + srct) * D, sizeof(uint16_t) * D);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* TurboQuant far tier: kernel semantics                                     */
/* ------------------------------------------------------------------------ */

/* foveated_2tier_turbo: csrc/kernels/foveated_attn.metal:559-767 with
 * dot_turbo_k (:486-521) and load_turbo_v (:531-552); q_rot = q.Pi^T and
 * q_sketch = q.S^T come from the host (csrc/foveated_attn.cpp:415-421) and
 * are passed here as the caller computed them.  fp64 throughout.
 *
 *   q           (B,Hq,D)   fp16 bits (near / decode scores use q * rsqrt(D))
 *   q_rot/q_sk  (B,Hq,D)   fp64
 *   near_k/v    (B,Hkv,Npad,D) fp16 bits; near_valid (Hkv)
 *   k_idx       (B,Hkv,F,D/4) 2-bit Lloyd-Max indices, dim 4j+i at bits 2i
 *   k_signs     (B,Hkv,F,D/8) QJL sign bits, dim 8j+i at bit i (1 -> +1)
 *   k_norm/k_gamma (B,Hkv,F) fp16 bits
 *   v_packed    (B,Hkv,F,D/4) 2-bit value codes, same packing as k_idx
 *   v_scale     (B,Hkv,F,D/32) fp16 bits, one scale per 32-dim group
 *   centroids   (4) fp32
 * Far score = (norm * sum q_rot*cb[idx] + (1.2533141/D) * gamma *
 * sum(+-1)*q_sketch) * rsqrt(D); far value = level[code] * scale with
 * levels {-1, -0.333333, 0.333333, 1}; split plan, gate, merge and spike
 * fields as orc_attend_kernel. */
ORC_API int orc_attend_turbo(int B, int Hq, int Hkv, int D, int Npad, int F, int n_dec,
                             const uint16_t* q, const double* q_rot, const double* q_sk,
                             const uint16_t* near_k, const uint16_t* near_v,
                             const uint32_t* near_valid, const uint8_t* k_idx,
                             const uint8_t* k_signs, const uint16_t* k_norm,
                             const uint16_t* k_gamma, const uint8_t* v_packed,
                             const uint16_t* v_scale, const float* centroids,
                             const uint16_t* dec_k, const uint16_t* dec_v, float spike_margin,
                             int split_size, int num_splits, int gate, double* out,
                             int32_t* flags, int32_t* tokens, double* max_far_out,
                             double* min_near_out) {
    if (Hkv <= 0 || Hq % Hkv != 0 || D <= 0 || D % 32 != 0) return -1;
    const int G = Hq / Hkv;
    const int s_total = Npad + F + n_dec;
    if (split_size <= 0 || num_splits <= 0) {
        int plan[3];
        orc_split_plan(s_total, plan);
        split_size = plan[0];
        num_splits = plan[1];
    }
    const float inv_sqrt_d = 1.0f / sqrtf((float)D);
    const float qjl = 1.2533141f / (float)D;
    const float levels[4] = {-1.0f, -0.333333f, 0.333333f, 1.0f};
    double* qreg = (double*)malloc(sizeof(double) * D);
    double* vv = (double*)malloc(sizeof(double) * D);
    double* racc = (double*)malloc(sizeof(double) * D);
    orc_state* sp = (orc_state*)malloc(sizeof(orc_state) * num_splits);
    double* accbuf = (double*)malloc(sizeof(double) * D * num_splits);
    if (!qreg || !vv || !racc || !sp || !accbuf) return -2;

    for (int b = 0; b < B; b++) {
        for (int hq = 0; hq < Hq; hq++) {
            const int kvh = hq / G;
            const int64_t bkv = (int64_t)b * Hkv + kvh;
            const int64_t o = (int64_t)b * Hq + hq;
            const double* qr = q_rot + o * D;
            const double* qs = q_sk + o * D;
            for (int d = 0; d < D; d++) qreg[d] = (double)(orc_h2f(q[o * D + d]) * inv_sqrt_d);
            for (int s = 0; s < num_splits; s++) {
                orc_state* st = &sp[s];
                st->m = -INFINITY;
                st->l = 0.0;
                st->acc = accbuf + (int64_t)s * D;
                for (int d = 0; d < D; d++) st->acc[d] = 0.0;
                st->min_near = INFINITY;
                st->max_far = -INFINITY;
                st->far_tok = -1;
                int g0 = s * split_size;
                int g1 = g0 + split_size < s_total ? g0 + split_size : s_total;
                int near0 = g0 < Npad ? g0 : Npad;
                int near1 = g1 < Npad ? g1 : Npad;
                int far0 = g0 > Npad ? (g0 - Npad < F ? g0 - Npad : F) : 0;
                int far1 = g1 > Npad ? (g1 - Npad < F ? g1 - Npad : F) : 0;
                int nf = Npad + F;
                int dec0 = g0 > nf ? (g0 - nf < n_dec ? g0 - nf : n_dec) : 0;
                int dec1 = g1 > nf ? (g1 - nf < n_dec ? g1 - nf : n_dec) : 0;
                int nv = (int)near_valid[kvh];
                int near_end = near1 < nv ? near1 : nv;
                for (int t = near0; t < near_end; t++) {
                    const uint16_t* kr = near_k + (bkv * Npad + t) * D;
                    const uint16_t* vr = near_v + (bkv * Npad + t) * D;
                    double sc = 0.0;
                    for (int d = 0; d < D; d++) sc += qreg[d] * (double)orc_h2f(kr[d]);
                    if (sc < st->min_near) st->min_near = sc;
                    for (int d = 0; d < D; d++) vv[d] = orc_h2f(vr[d]);
                    orc_accum(st, sc, vv, D);
                }
                for (int t = far0; t < far1; t++) {
                    const int64_t tok = bkv * F + t;
                    const uint8_t* ki = k_idx + tok * (D / 4);
                    const uint8_t* ks = k_signs + tok * (D / 8);
                    double mse = 0.0, sgn = 0.0;
                    for (int d = 0; d < D; d++) {
                        const int c = (ki[d >> 2] >> (2 * (d & 3))) & 3;
                        mse += qr[d] * (double)centroids[c];
                        sgn += ((ks[d >> 3] >> (d & 7)) & 1) ? qs[d] : -qs[d];
                    }
                    const double sc = ((double)orc_h2f(k_norm[tok]) * mse +
                                       (double)qjl * (double)orc_h2f(k_gamma[tok]) * sgn) *
                                      (double)inv_sqrt_d;
                    if (sc > st->max_far) { st->max_far = sc; st->far_tok = t; }
                    if (gate && sc < st->m - 16.0) continue;
                    const uint8_t* vp = v_packed + tok * (D / 4);
                    const uint16_t* vs = v_scale + tok * (D / 32);
                    for (int d = 0; d < D; d++) {
                        const int c = (vp[d >> 2] >> (2 * (d & 3))) & 3;
                        vv[d] = (double)levels[c] * (double)orc_h2f(vs[d >> 5]);
                    }
                    orc_accum(st, sc, vv, D);
                }
                for (int t = dec0; t < dec1; t++) {
                    const uint16_t* kr = dec_k + (bkv * n_dec + t) * D;
                    const uint16_t* vr = dec_v + (bkv * n_dec + t) * D;
                    double sc = 0.0;
                    for (int d = 0; d < D; d++) sc += qreg[d] * (double)orc_h2f(kr[d]);
                    if (sc < st->min_near) st->min_near = sc;
                    for (int d = 0; d < D; d++) vv[d] = orc_h2f(vr[d]);
                    orc_accum(st, sc, vv, D);
                }
            }
            double mg = -INFINITY, lg = 0.0, min_near = INFINITY, max_far = -INFINITY;
            int far_tok = -1;
            for (int d = 0; d < D; d++) racc[d] = 0.0;
            for (int s = 0; s < num_splits; s++) {
                orc_state* st = &sp[s];
                if (st->m == -INFINITY) continue;
                double mn = mg > st->m ? mg : st->m;
                double ag = mg > -INFINITY ? exp(mg - mn) : 0.0;
                double as = exp(st->m - mn);
                lg = ag * lg + as * st->l;
                for (int d = 0; d < D; d++) racc[d] = ag * racc[d] + as * st->acc[d];
                mg = mn;
                if (st->min_near < min_near) min_near = st->min_near;
                if (st->max_far > max_far) { max_far = st->max_far; far_tok = st->far_tok; }
            }
            double inv_l = lg > 0.0 ? 1.0 / lg : 0.0;
            for (int d = 0; d < D; d++) out[o * D + d] = racc[d] * inv_l;
            flags[o] = (max_far > min_near + (double)spike_margin) ? 1 : 0;
            tokens[o] = far_tok;
            if (max_far_out) max_far_out[o] = max_far;
            if (min_near_out) min_near_out[o] = min_near;
        }
    }
    free(qreg);
    free(vv);
    free(racc);
    free(sp);
    free(accbuf);
    return 0;
}
