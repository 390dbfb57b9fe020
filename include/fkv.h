/*
 * fkv.h -- C ABI of the MI355X (gfx950) FoveatedKV decode hot path.
 *
 * This is the drop-in boundary that replaces the reference's nanobind module
 * `foveated_ext` (samfurr/foveated_kv csrc/bindings.cpp:13-159).  Every
 * entry point takes plain pointers and sizes; device pointers are borrowed
 * (the caller owns them and keeps them alive for the call), `stream` is a
 * hipStream_t (NULL = the legacy default stream).  All work is enqueued
 * asynchronously on that stream unless stated otherwise.
 *
 * Errors: every int-returning function returns FKV_OK (0) on success and a
 * negative FKV_E* code otherwise; fkv_last_error() gives the message of the
 * calling thread's last failure.  No C++ exception crosses this boundary.
 * The reference raises std::runtime_error / silently ignores bad input in
 * the places noted per entry point; here the same conditions return codes.
 */
#ifndef FKV_H
#define FKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FKV_OK 0
#define FKV_EINVAL -1   /* bad argument / shape */
#define FKV_EHIP -2     /* HIP runtime error */
#define FKV_ENOMEM -3   /* device allocation failed */
#define FKV_EDATA -4    /* input data outside what the reference can produce */

/* most spiking far tokens a call reports per query head (fkv_attn_set_spike_k) */
#define FKV_MAX_SPIKE_K 32

/* element types accepted where noted */
#define FKV_F16 0
#define FKV_BF16 1
#define FKV_F32 2

/* ---------------------------------------------------------------------- */
/* library                                                                 */
/* ---------------------------------------------------------------------- */

/* Replaces foveated_ext.is_available (csrc/bindings.cpp:158-159): 1 when a
 * gfx950 device is visible to the HIP runtime, else 0. */
int fkv_is_available(void);
/* Message of the calling thread's last failed call ("" if none). */
const char* fkv_last_error(void);
/* ABI version (major*100 + minor). */
int fkv_version(void);

/* ---------------------------------------------------------------------- */
/* tier configuration (csrc/foveated_compress.h:92-98, mlx_foveated.py:111-169) */
/* ---------------------------------------------------------------------- */

typedef struct fkv_tier_config {
    double near_pct;           /* fraction of tokens kept in the fp16 near tier */
    int32_t n_sinks;
    int32_t window_size;
    double promo_headroom_pct; /* near headroom as a fraction of R_actual */
    int32_t promo_headroom_min;
    int32_t v_group;           /* far V INT4 scale / zero: 0 = one per token (the
                                  reference), 32 = one per 32-dim group */
    int32_t k_scale;           /* far K E4M3: 0 = unscaled (the reference), 1 = per
                                  (batch, head) scale amax/240 (fkv_compress_layer_ex) */
} fkv_tier_config;

typedef struct fkv_tiers {
    int32_t n_sinks, window, near_from_mid, far_count, r_actual, n_near_padded;
    int32_t mid_start, mid_end, near_mid_start, headroom;
} fkv_tiers;

/* Replaces MLXTierConfig.tier_boundaries (mlx_foveated.py:128-169) and its
 * C++ twin (csrc/foveated_compress.cpp:107-126).  Host-only, synchronous. */
int fkv_tier_boundaries(const fkv_tier_config* cfg, int32_t S, fkv_tiers* out);

/* ---------------------------------------------------------------------- */
/* compression (CompressHandle, csrc/foveated_compress.cpp:95-227)          */
/* ---------------------------------------------------------------------- */

/* Compress one layer: keys/values (B,H,S,D) contiguous in `in_dtype`
 * (converted to fp16 first, as astype(float16) at :129-130) into
 *   near_k, near_v   (B,H,Npad,D) fp16, rows >= R_actual zero  (compress_foveal)
 *   far_k            (B,H,F,D)    E4M3 codes                  (compress_fp8)
 *   far_v            (B,H,F,D/2)  INT4, even dim in low nibble (compress_int4)
 *   far_v_scale/zero (B,H,F)      fp16; (B,H,F,D/32) when cfg->v_group = 32
 *   near_valid       (H)          int32 = R_actual
 *   archive_k/v      (B,H,F,D)    fp16 copy of the far rows (may be NULL)
 * with Npad/F from fkv_tier_boundaries(cfg, S).  D must be 64 or 128.
 * One fused pass over K and V. */
int fkv_compress_layer(const fkv_tier_config* cfg, const void* keys, const void* values,
                       int32_t in_dtype, int32_t B, int32_t H, int32_t S, int32_t D,
                       void* near_k, void* near_v, uint8_t* far_k, uint8_t* far_v,
                       void* far_v_scale, void* far_v_zero, int32_t* near_valid,
                       void* archive_k, void* archive_v, void* stream);

/* Importance partition.  The reference partitions by recency
 * (mlx_foveated.py:128-169, 719-752); the benchmark configurations ask for
 * "sinks + window + top-importance middle", which importance = position
 * reproduces exactly.  importance (B,H,S) fp32 contiguous.  Per (b, h) the
 * near middle is the near_from_mid middle tokens of highest importance,
 * ties to the later token, NaN below every number, -0 == +0.  Writes
 *   near_idx (B,H,Npad) int32: sinks, chosen middle (ascending), window,
 *                              then -1 for the headroom slots
 *   far_idx  (B,H,F)    int32: the rest of the middle, ascending
 * with Npad/F from fkv_tier_boundaries(cfg, S).  One workgroup per (b, h):
 * an 8-pass radix select of the rank key, then a stable compaction. */
int fkv_partition_importance(const fkv_tier_config* cfg, const float* importance, int32_t B, int32_t H,
                             int32_t S, int32_t* near_idx, int32_t* far_idx, void* stream);

/* fkv_compress_layer from explicit index sets (as fkv_partition_importance
 * writes them): near slot s < R_actual is the row near_idx[b,h,s], far row
 * f is far_idx[b,h,f]; the archive holds the far rows in far_idx order.
 * Indices outside [0,S) give zero rows.  Same outputs and codecs as
 * fkv_compress_layer (which equals this with the recency index sets). */
int fkv_compress_layer_indexed(const fkv_tier_config* cfg, const void* keys, const void* values,
                               int32_t in_dtype, int32_t B, int32_t H, int32_t S, int32_t D,
                               const int32_t* near_idx, const int32_t* far_idx, void* near_k, void* near_v,
                               uint8_t* far_k, uint8_t* far_v, void* far_v_scale, void* far_v_zero,
                               int32_t* near_valid, void* archive_k, void* archive_v, void* stream);

/* Both compress entry points above in one, plus the benchmark's
 * per-head-scaled fp8 keys (no counterpart in the reference, whose keys are
 * encoded unscaled, csrc/kernels/foveated_compress.metal:39-66, 120-142):
 * near_idx / far_idx both NULL = fkv_compress_layer, both given =
 * fkv_compress_layer_indexed.  With cfg->k_scale = 1 each (batch, head)
 * gets scale = amax / 240 (fp32) over the finite values of its far keys (1
 * when amax is 0), written to far_k_scale (B,H) fp32, and its far keys are
 * encoded as Metal-encoder(fp16(key / scale)): the head's largest |key|
 * encodes to 0x77 (240, the top of the Metal encoder's 3-bit-mantissa
 * range: it emits exponent 15 only as the saturation code 0x7E = 448) and
 * scale = 1 gives the unscaled codes.  The keys
 * are read twice (scale, then encode).  far_k_scale may be NULL when
 * cfg->k_scale = 0.  fkv_compress_layer / _indexed return FKV_EINVAL for
 * cfg->k_scale = 1. */
int fkv_compress_layer_ex(const fkv_tier_config* cfg, const void* keys, const void* values, int32_t in_dtype,
                          int32_t B, int32_t H, int32_t S, int32_t D, const int32_t* near_idx,
                          const int32_t* far_idx, void* near_k, void* near_v, uint8_t* far_k, uint8_t* far_v,
                          void* far_v_scale, void* far_v_zero, float* far_k_scale, int32_t* near_valid,
                          void* archive_k, void* archive_v, void* stream);

/* ---------------------------------------------------------------------- */
/* fused attention handle (FoveatedHandle, csrc/foveated_attn.cpp:135-254)  */
/* ---------------------------------------------------------------------- */

typedef struct fkv_attn fkv_attn;

/* Copies the static tier arrays into a private device blob (re-laid out
 * for the gfx950 kernel), like FoveatedHandle's constructor (:135-162):
 *   near_k/near_v (B,Hkv,Na,D) in near_dtype (fp16/bf16/f32)
 *   far_k (B,Hkv,F,D) u8, far_v (B,Hkv,F,D/2) u8
 *   far_v_scale/zero (B,Hkv,F) in sz_dtype, near_valid (Hkv) int32
 * F may be 0.  Returns FKV_EDATA if far_k holds the E4M3 NaN codes
 * 0x7F/0xFF, which the reference encoder never emits.  Synchronous. */
int fkv_attn_create(fkv_attn** out, int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F,
                    const void* near_k, const void* near_v, int32_t near_dtype,
                    const uint8_t* far_k, const uint8_t* far_v, const void* far_v_scale,
                    const void* far_v_zero, int32_t sz_dtype, const int32_t* near_valid,
                    float spike_margin, void* stream);

/* Group-32 INT4 V variant of fkv_attn_create (the benchmark's
 * "fp8 K + INT4 V in group-32 packed layout"; the reference quantises V
 * per token, foveated_compress.metal:153-205, and this applies the same
 * quantiser to every 32-dim group).  Arguments as fkv_attn_create except
 *   far_v_scale/zero (B,Hkv,F,D/32) in sz_dtype, one pair per value group.
 * The returned handle is called, queried and destroyed with the
 * fkv_attn_* functions.  Synchronous. */
int fkv_attn_create_g32(fkv_attn** out, int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F,
                        const void* near_k, const void* near_v, int32_t near_dtype,
                        const uint8_t* far_k, const uint8_t* far_v, const void* far_v_scale,
                        const void* far_v_zero, int32_t sz_dtype, const int32_t* near_valid,
                        float spike_margin, void* stream);

/* TurboQuant handle: replaces TurboFoveatedHandle's constructor
 * (csrc/foveated_attn.cpp:365-405, blob builder :306-363).  Same near
 * tier and near_valid as fkv_attn_create; the far tier is
 *   k_idx   (B,Hkv,F,D/4) u8  2-bit Lloyd-Max indices, dim 4j+i at bits 2i
 *   k_signs (B,Hkv,F,D/8) u8  QJL sign bits, dim 8j+i at bit i (1 = +1)
 *   k_norm, k_gamma (B,Hkv,F) in nz_dtype (stored as fp16)
 *   v_packed (B,Hkv,F,D/4) u8 2-bit value codes, packed like k_idx
 *   v_scale (B,Hkv,F,D/32) in nz_dtype (stored as fp16)
 * Pi, S (D,D) and centroids (4) are fp32 device arrays (the rotation, the
 * QJL matrix and the Lloyd-Max centroids); the handle keeps its own
 * copies.  The returned handle is called, queried and destroyed with the
 * fkv_attn_* functions; each call first rotates and sketches the query
 * (q.Pi^T, q.S^T, foveated_attn.cpp:415-421).  Synchronous. */
int fkv_turbo_create(fkv_attn** out, int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F,
                     const void* near_k, const void* near_v, int32_t near_dtype, const uint8_t* k_idx,
                     const uint8_t* k_signs, const void* k_norm, const void* k_gamma, const uint8_t* v_packed,
                     const void* v_scale, int32_t nz_dtype, const int32_t* near_valid, const float* Pi,
                     const float* S, const float* centroids, float spike_margin, void* stream);

/* TurboQuant compression on the GPU (src/foveated_kv/turbo_quantize.py:
 * 25-91): keys (n_tokens, D) in dtype -> out_idx (n_tokens, D/4) u8,
 * out_signs (n_tokens, D/8) u8, out_norm / out_gamma (n_tokens) fp16;
 * Pi, S (D,D), centroids (4), boundaries (3) fp32 device arrays.  fp32
 * arithmetic; a code whose rotated coordinate lies within fp32 rounding of
 * a boundary (or a sign whose projection lies within rounding of 0) can
 * differ from another fp32 evaluation order.  Synchronous (reads the
 * centroids). */
int fkv_turbo_compress_keys(const void* keys, int32_t dtype, int64_t n_tokens, int32_t D, const float* Pi,
                            const float* S, const float* centroids, const float* boundaries, uint8_t* out_idx,
                            uint8_t* out_signs, void* out_norm, void* out_gamma, void* stream);

/* turbo_compress_values (turbo_quantize.py:139-178): values (n_tokens, D)
 * -> out_packed (n_tokens, D/4) u8 2-bit codes, out_scale (n_tokens, D/32)
 * fp16, one scale per 32 dims; codes round half to even.  Asynchronous. */
int fkv_turbo_compress_values(const void* values, int32_t dtype, int64_t n_tokens, int32_t D, uint8_t* out_packed,
                              void* out_scale, void* stream);

/* Replaces FoveatedHandle::operator() (:164-240) and, for a TurboQuant
 * handle, TurboFoveatedHandle::operator() (:407-491): query (B,Hq,1,D) in
 * q_dtype, decode_k/v (B,Hkv,n_decode,D) fp16 (NULL when n_decode == 0).
 * Writes out (B,Hq,D) fp16, spike_flags/spike_tokens (B,Hq) int32.
 *
 * Workspace: a handle's first call (of any fkv_attn_call* variant)
 * allocates the handle's split workspace for that call's Hq, large enough
 * for every decode length; no later call allocates or frees anything, so
 * a HIP graph captured around a call stays valid for the handle's life.
 * Later calls with a different Hq return FKV_EINVAL (one handle serves one
 * query-head count, as a model layer does).  The first call is therefore
 * not capturable.  One handle owns one workspace and one set of split
 * arrival counters, which every call reuses: an eager call on another
 * stream than the handle's last eager call first waits (hipStreamWaitEvent)
 * for that call's work, so calls on one handle never overlap.  Calls under
 * graph capture neither wait nor record: the replays of a captured graph,
 * and eager calls beside them, are ordered by the caller. */
int fkv_attn_call(fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq,
                  const void* decode_k, const void* decode_v, int32_t n_decode, void* out,
                  int32_t* spike_flags, int32_t* spike_tokens, void* stream);

/* fkv_attn_call on a decode buffer with a row stride (no counterpart in the
 * reference, whose decode buffer is re-concatenated each step,
 * mlx_foveated.py:404-428): decode_k/v (B,Hkv,row_stride,D) fp16, rows
 * [0, n_decode) valid, row_stride >= n_decode.  A growing decode buffer is
 * attended to in place, without a per-call copy. */
int fkv_attn_call_strided(fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq, const void* decode_k,
                          const void* decode_v, int32_t n_decode, int32_t row_stride, void* out,
                          int32_t* spike_flags, int32_t* spike_tokens, void* stream);

/* fkv_attn_call that allocates nothing.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory during a call (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, outputs and kernels as fkv_attn_call; the
 * call's split records, arrival counters and fp16 query copy live in one
 * fixed 8 MiB device array per GPU instead of the handle's workspace, so
 * neither this call nor its first use allocates or frees anything.  Calls
 * whose launch plan needs more than the array holds (64 KiB of arrival
 * counters for at most 16384 rows, then the fp16 query copy, then rows x
 * splits x records per split x heads per row x (8 + D) floats of split
 * records, fkv_attn_plan out[1] x out[2] x out[7] x min(out[0], G); C3 at
 * batch 8 needs 2.25 MiB: 64 rows x 4 splits x 4 wave records x 4 heads x
 * 136 floats, C5 1.14 MiB) return FKV_EINVAL, as does a call whose handle's
 * device is not current, or, with spike_k > 1, a handle whose top-K
 * selection buffers do not exist yet (fkv_attn_set_spike_k).  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams, two threads) race and must be ordered by the caller. */
int fkv_attn_call_noalloc(fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq, const void* decode_k,
                          const void* decode_v, int32_t n_decode, void* out, int32_t* spike_flags,
                          int32_t* spike_tokens, void* stream);

/* The launch plan of one call (host only, no GPU; no counterpart in the
 * reference, whose split sizing is foveated_attn.cpp:26-38): for a handle of
 * shape (B, Hkv, D, Na, F) and far format fmt (0: fp8 K / per-token V, 1:
 * TurboQuant, 2: fp8 K / group-32 V) called with Hq query heads and n_decode
 * decode rows, aiming at target_wgs workgroups, writes out[0] query heads per
 * workgroup row, out[1] rows, out[2] splits per row, out[3] split-partial
 * floats the call uses, out[4] floats the handle's workspace holds, out[5]
 * arrival counters it holds, out[6] waves per workgroup, out[7] split records
 * per split (one per wave, or 1 when a split merges its waves in LDS).  An
 * introspection hook: tests check that no decode length needs more
 * workspace than the first call allocates. */
int fkv_attn_plan(int32_t B, int32_t Hkv, int32_t D, int32_t Na, int32_t F, int32_t Hq, int32_t n_decode,
                  int32_t target_wgs, int32_t fmt, int64_t* out);

/* The attention kernel's far-tile plan for one row (host only, no GPU): wave
 * w of n_waves streams far tiles f0[w] + u * fs[w], u < nf[w].  near_weight
 * is a near tile's weight in bytes (256 * D for one head quad per row, half
 * for more), far_rec a far record's bytes, turbo nonzero for the TurboQuant
 * layout.  No counterpart in the reference (its split is per q head, not per
 * wave): an introspection hook so tests can check every far tile is planned
 * exactly once. */
int fkv_far_plan(int32_t n_waves, int32_t near_plan, int32_t nt_far, int64_t near_weight, int64_t far_rec,
                 int32_t turbo, int32_t* f0, int32_t* fs, int32_t* nf);

/* The workgroup -> XCD dispatch rule the handle's split merge relies on (no
 * counterpart in the reference, whose Metal kernel has no merge across
 * dies): *xcd_mod = X where the device deals a dispatch's workgroups to its X
 * XCDs round-robin by linear index (checked once per device when its first
 * handle is created), so that the splits of one row can merge in one XCD's
 * L2; 0 when the rule did not hold or the handle was created with
 * FKV_XCD_LOCAL=0 (the merge then goes through memory).  Host only. */
int fkv_attn_dispatch_info(const fkv_attn* h, int32_t* xcd_mod);

/* Checks the dispatches since the last check against that rule (no
 * counterpart in the reference): every split record carries the XCD that
 * wrote it, and an XCD-local merge raises the handle's watch flag when a
 * record of its row came from another XCD (or is a stale one another XCD
 * left behind).  Synchronises `stream`, then reads the handle's flag and
 * arrival counters and those of the device's no-alloc scratch:
 * *violations = flags raised plus counters left nonzero (a broken pattern
 * can also split a row's arrival count across L2s, so that no workgroup
 * merges the row or re-arms its counter).  Any violation switches the
 * handle to the merge through memory (fkv_attn_dispatch_info then reports
 * 0) and clears the counters; the outputs of the violating dispatches may
 * be stale. */
int fkv_attn_dispatch_check(fkv_attn* h, int32_t* violations, void* stream);

/* Host-only helpers of the two checks above, for tests: fkv_xcd_rule_fit
 * sets *xcd_mod = X and *offset = c when xcc[i] = lo + (c + i) mod X for
 * every i < n (lo the smallest id, X the id span), else 0 and 0;
 * fkv_xcd_watch_violations returns the violations an array [flag, arrival
 * counter of rows 0 .. rows-1] holds (a raised flag, counters not zero). */
int fkv_xcd_rule_fit(const uint32_t* xcc, int32_t n, int32_t* xcd_mod, int32_t* offset);
int32_t fkv_xcd_watch_violations(const uint32_t* words, int32_t rows);

/* Per-workgroup phase timestamps of the attention kernels (no counterpart in
 * the reference; a measurement hook): only a library built with
 * -DFKV_PHASE_STAMPS records them (make STAMPS=1), any other returns
 * FKV_EINVAL.  Copies the first n_wgs workgroups' 64 slots (100 MHz clock
 * values; slot 63 = the workgroup's XCD; the slots are listed in
 * fkv_attn_kernel.h) of the last launches to out, then zeroes them when
 * clear is set.  Synchronous. */
int fkv_phase_stamps(uint64_t* out, int32_t n_wgs, int32_t clear);

/* fkv_attn_call with the decode-buffer length in device memory, for callers
 * that capture decode steps in a HIP graph (no counterpart in the
 * reference): decode_k/v (B,Hkv,capacity,D) fp16, rows [0, *n_decode_dev)
 * valid; the kernel reads *n_decode_dev (clamped to [0, capacity]). */
int fkv_attn_call_dev(fkv_attn* h, const void* query, int32_t q_dtype, int32_t Hq, const void* decode_k,
                      const void* decode_v, const int32_t* n_decode_dev, int32_t capacity, void* out,
                      int32_t* spike_flags, int32_t* spike_tokens, void* stream);

/* Per-head-scaled fp8 keys for an fp8 handle (fkv_attn_create /
 * fkv_attn_create_g32; no counterpart in the reference, whose keys are
 * unscaled): k_scale (B,Hkv) fp32 device array, as fkv_compress_layer_ex
 * writes it; a far key is then decode(code) * scale.  The kernel applies
 * the scale to the far scores (one multiply folded into 1/sqrt(D)), so the
 * far tile's arithmetic is unchanged.  A new handle's scales are 1.  Returns
 * FKV_EDATA for a scale that is not a positive finite number, FKV_EINVAL for
 * a TurboQuant handle.  Synchronous. */
int fkv_attn_set_k_scale(fkv_attn* h, const float* k_scale, void* stream);

/* Top-K spike tokens (the benchmark's "up to 32 far tokens per head per
 * step"; no counterpart in the reference, whose kernel reports one token per
 * query head, csrc/kernels/foveated_attn.metal:323-327, 427-430).  With
 * spike_k = K in [2, FKV_MAX_SPIKE_K] every later call writes
 *   spike_flags  (B,Hq)   the number of far tokens whose score exceeds the
 *                         head's min_near + margin, at most K (0 or 1 for K =
 *                         1: the reference's flag);
 *   spike_tokens (B,Hq,K) those tokens' far-local indices in descending
 *                         score order, ties to the smaller index; entry 0 is
 *                         the first-index argmax of the far scores when no
 *                         token spikes (the reference's token), other
 *                         entries past the count -1.
 * A second kernel rescores the far tiles whose maximum can hold a spike (the
 * attention kernel stores each far tile's per-head maximum), so with sparse
 * spikes the extra work is a few tiles per head.  K = 1 (the default) is the
 * reference's single token, with no extra work.  TurboQuant handles take K
 * = 1 only.  Allocates the selection's buffers when the handle's workspace
 * exists (else its next call does); fkv_attn_call_noalloc with K > 1 needs
 * them to exist.  Host only. */
int fkv_attn_set_spike_k(fkv_attn* h, int32_t spike_k);

/* Replaces get_blob_info (:242-254): where promotions land. */
typedef struct fkv_blob_info {
    void* blob;               /* device base pointer */
    uint64_t blob_bytes;
    uint64_t near_k_offset;   /* [B*Hkv][Na_pad/64][D/8][64][8] fp16 tiles:
                                 token t, dim d at ((t/64)*D/8 + d/8)*512 + (t%64)*8 + d%8 */
    uint64_t near_v_offset;   /* [B*Hkv][Na_pad/64] tiles of 64*D fp16: token t,
                                 dim d, x = (d/64)*16 + (t%64)/4, at
                                 (t/64)*64*D + (x/2)*512 + (d%64)*8 + (x%2)*4 + t%4 */
    uint64_t near_valid_offset; /* (Hkv) uint32 */
    int32_t n_near_alloc;     /* Na: near slots per head incl. headroom */
    int32_t n_far;
    int32_t B, H_kv, D;
} fkv_blob_info;
int fkv_attn_blob_info(const fkv_attn* h, fkv_blob_info* out);

/* Copies near_valid (Hkv uint32) to host memory (synchronous on stream). */
int fkv_attn_read_near_valid(const fkv_attn* h, uint32_t* host_out, void* stream);

void fkv_attn_destroy(fkv_attn* h);

/* Decodes n (multiple of 4) E4M3 codes to fp16 with the converter the fused
 * kernel uses (gfx950 v_cvt_scalef32_pk_f16_fp8).  Replaces the reference's
 * decode LUT (csrc/kernels/foveated_attn.metal:237-253) for verification:
 * equal on every code the reference encoder emits. */
int fkv_e4m3_decode(const uint8_t* codes, void* out_f16, int64_t n, void* stream);

/* GPU side of one promotion batch (csrc/promotion_pipeline.cpp:192-241):
 * on `stream`, writes n exact fp16 rows into near-tier slots and then, after
 * them, raises near_valid[head] to slot + 1 with device-scope atomics.
 * head_slot: device int32 [n][2] = (kv head, slot); rows_k / rows_v: device
 * fp16 [n][row_batches][D], the row of batches 0..row_batches-1 (batches
 * above keep their slot unchanged, like the reference's batch-0-only copy).
 * Records whose head or slot fall outside the blob are skipped. */
int fkv_attn_promote_rows(fkv_attn* h, int32_t n, const int32_t* head_slot, const void* rows_k,
                          const void* rows_v, int32_t row_batches, void* stream);

/* The blob's near tier back to row-major (B, Hkv, Na, D) fp16 device
 * buffers (either may be NULL): what the kernel attends to, promotions
 * included. */
int fkv_attn_export_near(const fkv_attn* h, void* near_k_out, void* near_v_out, void* stream);

/* ---------------------------------------------------------------------- */
/* promotion pipeline (PromotionPipeline, csrc/promotion_pipeline.h:75-141)  */
/* ---------------------------------------------------------------------- */

typedef struct fkv_promoter fkv_promoter;

/* PromotionStats (promotion_pipeline.h:42-49). */
typedef struct fkv_promoter_stats {
    uint64_t spikes_detected, spikes_queued, spikes_deduplicated, spikes_cooled_down;
    uint64_t promotions_completed, promotions_headroom_full;
} fkv_promoter_stats;

/* PromotionPipeline(n_layers, cooldown_steps=5, max_per_drain=8)
 * (bindings.cpp:43-47).  Host only: no GPU work until the first flush. */
int fkv_promoter_create(int32_t n_layers, int32_t cooldown_steps, int32_t max_per_drain, fkv_promoter** out);

/* Tokens per query head the drains take (no counterpart in the reference,
 * whose drain takes one, promotion_pipeline.cpp:120-172): with spike_k = K in
 * [2, FKV_MAX_SPIKE_K], spike_flags hold spike counts and spike_tokens are
 * (B*Hq, K), as fkv_attn_call writes them for a handle with the same
 * spike_k.  The first flagged query head of a KV head (GQA dedup) then hands
 * up to K tokens, in order, through the position dedup and the archive
 * lookup; the cooldown applies to the KV head once per drain, the per-call
 * budget max_per_drain counts tokens and is checked before each token.  A
 * KV head therefore promotes at most K rows per drain.  K = 1 (the default)
 * is the reference's drain.  Host only. */
int fkv_promoter_set_spike_k(fkv_promoter* p, int32_t spike_k);

/* register_archive (promotion_pipeline.cpp:45-83) from host rows
 * [B_arc][Hkv][S_arc][D] fp16 and archive_idx [Hkv][S_arc] int32 (global
 * position of each archive row).  copy_to_pinned: copy the rows into
 * pinned host memory owned by the pipeline (else the pointers are
 * borrowed and must stay valid). */
int fkv_promoter_register_archive(fkv_promoter* p, int32_t layer, const void* k, const void* v, int32_t B_arc,
                                  int32_t Hkv, int32_t S_arc, int32_t D, const int32_t* archive_idx,
                                  int32_t copy_to_pinned);

/* register_archive with the rows [B_arc][Hkv][S_arc][D] fp16 already in
 * device memory (e.g. the compress kernel's archive output), borrowed: they
 * must stay valid while the layer is registered.  No counterpart in the
 * reference, whose archive is host (on its platform, unified) memory: on
 * MI355X the device drain reads a pinned host archive over PCIe, while HBM
 * holds a model's whole archive (C5: 241 MB per layer); at C5 with 32
 * tokens per head the drain kernel takes 6.4 us instead of 6.6.  The device
 * drain reads the rows in place; the host drain copies them device to
 * device.  D must be a multiple of 8. */
int fkv_promoter_register_archive_device(fkv_promoter* p, int32_t layer, const void* k, const void* v, int32_t B_arc,
                                         int32_t Hkv, int32_t S_arc, int32_t D, const int32_t* archive_idx);

/* register_archive from the reference's on-disk archive files
 * (disk_archive.py:127-185: (Hkv, S_arc, D) fp16 raw, batch 0), read into
 * pinned host memory.  An unreadable file leaves the layer without an
 * archive (drain is then a no-op for it, as in the reference). */
int fkv_promoter_register_archive_files(fkv_promoter* p, int32_t layer, const char* path_k, const char* path_v,
                                        int32_t Hkv, int32_t S_arc, int32_t D, const int32_t* archive_idx);

/* register_blob (promotion_pipeline.h:95): the layer's attention handle.
 * Reads its near_valid once (synchronous on stream) into the pipeline's
 * host mirror; the pipeline must then be the only writer of near_valid. */
int fkv_promoter_register_handle(fkv_promoter* p, int32_t layer, fkv_attn* h, void* stream);

/* drain_spikes (promotion_pipeline.cpp:99-175), host only: spike_flags /
 * spike_tokens (B*Hq) and far_idx (B, Hkv, N_far) are host int32 arrays.
 * Returns the number of records queued (>= 0); invalid layers or a layer
 * without archive queue nothing, as in the reference. */
int fkv_promoter_drain(fkv_promoter* p, int32_t layer, const int32_t* spike_flags, const int32_t* spike_tokens,
                       const int32_t* far_idx, int32_t B, int32_t Hq, int32_t Hkv, int32_t N_far, int32_t step);

/* Device-side drain + promotion.  No counterpart in the reference, whose
 * drain runs on the host after reading the spike outputs back: the same
 * filter as fkv_promoter_drain (scan order, GQA dedup, cooldown, position
 * dedup, budget) and the same commit as the flush (rows of every archive
 * batch into the next headroom slot, then the near_valid bump), as one
 * kernel on `stream` reading spike_flags / spike_tokens (B*Hq) and far_idx
 * (B, Hkv, N_far) int32 in device memory and the archive rows from the
 * pipeline's pinned host copy.  No host synchronisation: the next launch on
 * `stream` sees the promoted rows.  For callers that keep a decode step on
 * the GPU.  Needs a registered handle and an archive registered with
 * copy_to_pinned (or from files); the first call per layer allocates (not
 * capturable).  A layer is drained either here or by fkv_promoter_drain:
 * the first drain on a layer fixes which, the other then returns
 * FKV_EINVAL for that layer (registering its handle again resets this);
 * fkv_promoter_near_valid reads a device-drained layer's near_valid from
 * the blob (synchronising).  Statistics accumulate on the device and
 * fkv_promoter_get_stats adds them (synchronising).
 * step_dev (may be NULL): the decode step is read from this device int32
 * instead of `step` (a graph-captured step keeps its counter on the GPU).
 * advance_step (needs step_dev): once the drain has read the step, the
 * stream's work stores step + 1 into *step_dev, on every successful call,
 * so a captured decode step needs no separate counter update; without
 * step_dev it returns FKV_EINVAL. */
int fkv_promoter_drain_device(fkv_promoter* p, int32_t layer, const int32_t* spike_flags,
                              const int32_t* spike_tokens, const int32_t* far_idx, int32_t B, int32_t Hq,
                              int32_t Hkv, int32_t N_far, int32_t step, int32_t* step_dev, int32_t advance_step,
                              void* stream);

/* Queued records (not yet flushed): returns their count and copies up to
 * max_records of them as int32 [layer, head, archive row, position]. */
int fkv_promoter_pending(const fkv_promoter* p, int32_t* out_records, int32_t max_records);

/* The worker's job (promotion_pipeline.cpp:192-241) as stream-ordered GPU
 * work on the pipeline's side stream: assign headroom slots (full headroom
 * is counted and skipped), gather the rows from the pinned archive, one
 * hipMemcpyAsync, fkv_attn_promote_rows per layer.  Returns immediately. */
int fkv_promoter_flush(fkv_promoter* p);

/* Make `stream` wait for the last flushed promotion of `layer` (call before
 * the layer's next attention launch: the rows and the new near_valid are
 * then visible together). */
int fkv_promoter_order(fkv_promoter* p, int32_t layer, void* stream);
int fkv_promoter_synchronize(fkv_promoter* p);
int fkv_promoter_get_stats(const fkv_promoter* p, fkv_promoter_stats* out);
/* A layer's near_valid (returns Hkv, copies up to n): the host mirror for a
 * host-drained layer, the blob's words for a device-drained one. */
int fkv_promoter_near_valid(const fkv_promoter* p, int32_t layer, uint32_t* out, int32_t n);
/* stop() + destructor (promotion_pipeline.cpp:30-38, 243-248). */
void fkv_promoter_destroy(fkv_promoter* p);

/* Benchmark utility with no counterpart in the reference: streams `bytes`
 * (a multiple of 16) from device buffer `buf` with 16-byte lane loads,
 * `unroll` (1, 2, 4, 8) loads in flight per lane, optionally non-temporal,
 * on `blocks` workgroups of 256 threads; writes one XOR fold per wave to
 * `out` (blocks*4 uint32).  Measures the device's practical HBM read
 * ceiling for the roofline of the attention kernel. */
int fkv_hbm_read_probe(const void* buf, int64_t bytes, int32_t unroll, int32_t nontemporal, int32_t blocks,
                       uint32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FKV_H */
