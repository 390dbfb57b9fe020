// Promotion pipeline: the spike drain filter (host) and the GPU side that
// copies exact fp16 rows from a host-pinned archive into near-tier headroom.
//
// Replaces the reference's PromotionPipeline (csrc/promotion_pipeline.h:75-141,
// csrc/promotion_pipeline.cpp:99-248).  The drain filter keeps the
// reference's semantics exactly: scan (batch, query head) in order until the
// per-call budget is reached; the first flagged query head of each KV head is
// the only candidate for that KV head in the call (GQA dedup); a per-(layer,
// KV head) cooldown in steps; never promote the same (layer, KV head,
// position) twice; far-local token -> global position -> archive-local row.
//
// The reference's worker thread memcpy's rows into unified memory and bumps
// near_valid[h] with a release store.  On MI355X the same commit protocol is
// stream-ordered device work: fkv_promoter_flush assigns headroom slots from
// a host mirror of near_valid (the pipeline is the only writer), gathers the
// rows into pinned staging, issues one hipMemcpyAsync on a side stream and
// then fkv_attn_promote_rows (row scatter, then the near_valid bump ordered
// after it).  fkv_promoter_order makes a compute stream wait for a layer's
// last promotion, so the next dispatch sees the rows and the new count
// together ("visible at the next dispatch", promotion_pipeline.cpp:236-237).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "fkv_attn.h"
#include "fkv_common.h"
#include "../../include/fkv.h"

using fkv::check_hip;
using fkv::set_error;

namespace {

struct Archive {
    const uint16_t* k = nullptr;  // [B_arc][Hkv][S_arc][D] fp16 (host, or device memory when `device`)
    const uint16_t* v = nullptr;
    void* owned_k = nullptr;  // pinned copies owned by the pipeline
    void* owned_v = nullptr;
    bool device = false;      // rows in device memory, borrowed (fkv_promoter_register_archive_device)
    int B = 0, Hkv = 0, S = 0, D = 0;
    std::vector<std::unordered_map<int32_t, int32_t>> pos_to_local;  // [Hkv]: position -> archive row
};

struct Record {
    int32_t layer, head, arc_local, position;
};

// Device-side drain state of one layer (fkv_promoter_drain_device)
struct DevDrain {
    int32_t* last_step = nullptr;     // [Hkv], kNoStep until the first candidate
    uint32_t* promoted = nullptr;     // [Hkv][words]: positions already promoted
    int32_t* pos_to_local = nullptr;  // [Hkv][P]: position -> archive row, -1 if none
    int P = 0, words = 0;
    const uint16_t* ark = nullptr;    // device views of the pinned archive rows
    const uint16_t* arv = nullptr;
};

constexpr int32_t kNoStep = INT32_MIN;
enum : uint8_t { kDrainNone = 0, kDrainHost = 1, kDrainDevice = 2 };
constexpr int kMaxDrainHeads = 256;

}  // namespace

struct fkv_promoter {
    int n_layers = 0, cooldown = 5, max_per_drain = 8;
    // spiking tokens a drain takes per query head (fkv_promoter_set_spike_k;
    // 1 = the reference's single token)
    int spike_k = 1;
    std::vector<Archive> arch;
    std::vector<fkv_attn*> handles;
    std::vector<std::vector<uint32_t>> mirror;  // host copy of each layer's near_valid
    std::vector<int> n_alloc;                   // near slots per head, per layer
    // per layer: which drain has committed into its blob (the host drain keeps
    // `mirror` current, the device drain writes near_valid in the blob only),
    // so the two are never mixed on one layer
    std::vector<uint8_t> mode;
    std::unordered_set<uint64_t> promoted;
    std::unordered_map<uint32_t, int> last_step;
    std::vector<Record> queue;
    fkv_promoter_stats stats{};
    // GPU side (created on first flush)
    hipStream_t side = nullptr;
    std::vector<hipEvent_t> done;      // per layer: last promotion on the side stream
    std::vector<uint8_t> has_done;
    hipEvent_t staged = nullptr;       // last H2D copy out of the pinned staging
    bool staged_pending = false;
    uint8_t* stage_h = nullptr;        // pinned host staging
    uint8_t* stage_d = nullptr;        // device staging
    size_t stage_cap = 0;
    // device drain
    std::vector<DevDrain> dev;
    unsigned long long* dstats = nullptr;  // 6 counters, fkv_promoter_stats order
};

namespace {

// Forget a layer's device-drain state (its archive is being replaced).
void free_dev_drain(fkv_promoter* p, int layer) {
    if (p->dev.empty() || !p->dev[layer].last_step) return;
    (void)hipDeviceSynchronize();  // a queued drain may still read it
    DevDrain& d = p->dev[layer];
    (void)hipFree(d.last_step);
    (void)hipFree(d.promoted);
    (void)hipFree(d.pos_to_local);
    d = DevDrain();
}

void free_archive(Archive& a) {
    if (a.owned_k) (void)hipHostFree(a.owned_k);
    if (a.owned_v) (void)hipHostFree(a.owned_v);
    a = Archive();
}

int build_positions(Archive& a, const int32_t* archive_idx) {
    a.pos_to_local.assign(a.Hkv, {});
    if (!archive_idx) return FKV_OK;
    for (int h = 0; h < a.Hkv; h++) {
        auto& m = a.pos_to_local[h];
        m.reserve((size_t)a.S);
        for (int i = 0; i < a.S; i++) m[archive_idx[(int64_t)h * a.S + i]] = i;
    }
    return FKV_OK;
}

int ensure_gpu(fkv_promoter* p) {
    if (p->side) return FKV_OK;
    int rc = check_hip(hipStreamCreateWithFlags(&p->side, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    if (!rc) rc = check_hip(hipEventCreateWithFlags(&p->staged, hipEventDisableTiming), "hipEventCreate");
    if (!rc) {
        p->done.assign(p->n_layers, nullptr);
        p->has_done.assign(p->n_layers, 0);
        for (int l = 0; l < p->n_layers && !rc; l++)
            rc = check_hip(hipEventCreateWithFlags(&p->done[l], hipEventDisableTiming), "hipEventCreate");
    }
    return rc;
}

int ensure_staging(fkv_promoter* p, size_t bytes) {
    if (bytes <= p->stage_cap) return FKV_OK;
    if (p->staged_pending) {
        if (int rc = check_hip(hipEventSynchronize(p->staged), "hipEventSynchronize")) return rc;
        p->staged_pending = false;
    }
    // the device staging may still be read by queued promote kernels
    if (int rc = check_hip(hipStreamSynchronize(p->side), "hipStreamSynchronize")) return rc;
    if (p->stage_h) (void)hipHostFree(p->stage_h);
    if (p->stage_d) (void)hipFree(p->stage_d);
    p->stage_h = nullptr;
    p->stage_d = nullptr;
    p->stage_cap = 0;
    size_t cap = 64 * 1024;
    while (cap < bytes) cap *= 2;
    if (int rc = check_hip(hipHostMalloc((void**)&p->stage_h, cap, hipHostMallocDefault), "hipHostMalloc(staging)"))
        return rc;
    if (int rc = check_hip(hipMalloc((void**)&p->stage_d, cap), "hipMalloc(staging)")) return rc;
    p->stage_cap = cap;
    return FKV_OK;
}

inline size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }

}  // namespace


namespace {

struct DrainArgs {
    const int32_t* flags;
    const int32_t* tokens;
    const int32_t* far_idx;
    int B, Hq, Hkv, N_far, step, cooldown, budget;
    int spike_k;        // tokens per query head (tokens is (B*Hq, spike_k))
    int32_t* step_dev;  // when set, the step is read here
    int advance;        // then step + 1 is stored there once every thread has read it
    int32_t* last_step;
    uint32_t* promoted;
    const int32_t* pos_to_local;
    int P, words;
    const uint16_t* ark;
    const uint16_t* arv;
    int arc_B, arc_S;
    fkv::BlobLayout L;
    uint8_t* blob;
    unsigned long long* stats;
};

// The drain filter (promotion_pipeline.cpp:99-175) and the promotion
// (:192-241) of one layer as one workgroup, with the sequential scan
// restated in parallel.  The scan visits (batch, query head) in order, keeps
// only the first spike of each KV head (its GQA dedup) and hands its tokens
// (one, or with spike_k > 1 up to spike_k in descending score order) through
// the position dedup and the archive lookup until `budget` tokens are
// queued.  Each KV head's state (last promotion step, promoted bitmap,
// near_valid) is touched only by its own first spike, and its tokens are
// distinct positions, so every head's outcome -- cooled down, or per token
// out of range, duplicate, no archived row, queued -- is independent of the
// others; the scan's budget stop then becomes a prefix sum: a head is
// processed iff the heads before it in scan order would queue fewer than
// `budget` tokens, and it queues at most the rest of the budget.  Within a
// head the scan stops at the token before which `allow` tokens are queued,
// so a token is reached iff fewer than `allow` of the head's earlier tokens
// are queued: a prefix count again.  Threads: one per (batch, query head) to
// find each head's first spike; with spike_k > 1 (TOPK) one per (KV head,
// token) for the token's outcome, one per KV head for the budget prefix, its
// cooldown and its counts, one per (KV head, token) again to mark the
// reached tokens' positions and record the queued ones' archive rows; with
// spike_k = 1 one per KV head for all of it; then all threads copy the
// exact fp16 rows of every archive batch (pinned host or device memory)
// into the assigned headroom slots, all heads' rows in one loop; the
// near_valid bumps are written last (the next launch on the stream sees
// rows and counts together).  A head's records take the slots from its
// near_valid on, in token order.
enum : int { kTokSkip = 0, kTokDup, kTokMarked, kTokQueued };

// The outcome of one token of KV head hkv's first spike (f: its flat
// (batch, query head) index); pos / arc / bit are set for the last three.
__device__ inline int drain_token(const DrainArgs& a, int f, int hkv, int j, int& pos, int& arc, uint32_t& bit,
                                  int64_t& widx) {
    const int fl = a.tokens[(int64_t)f * a.spike_k + j];
    if (fl < 0 || fl >= a.N_far) return kTokSkip;
    const int32_t p = a.far_idx[((int64_t)(f / a.Hq) * a.Hkv + hkv) * a.N_far + fl];
    if (p < 0 || p >= a.P) return kTokSkip;
    pos = p;
    widx = (int64_t)hkv * a.words + (p >> 5);
    bit = 1u << (p & 31);
    if (a.promoted[widx] & bit) return kTokDup;
    arc = a.pos_to_local[(int64_t)hkv * a.P + p];
    return arc >= 0 ? kTokQueued : kTokMarked;
}

template <bool TOPK>
__global__ __launch_bounds__(256) void drain_promote_kernel(DrainArgs a) {
    __shared__ int first[kMaxDrainHeads];
    __shared__ int nq[kMaxDrainHeads];                  // tokens each head would queue
    __shared__ int n_rec[kMaxDrainHeads], slot0[kMaxDrainHeads];
    __shared__ int rec_arc[kMaxDrainHeads][TOPK ? FKV_MAX_SPIKE_K : 1];
    __shared__ unsigned cnt[6];  // detected, queued, deduplicated, cooled down, records, headroom full
    const int tid = threadIdx.x;
    for (int i = tid; i < kMaxDrainHeads; i += blockDim.x) {
        first[i] = INT_MAX;
        nq[i] = 0;
        n_rec[i] = 0;
    }
    if (tid < 6) cnt[tid] = 0;
    __syncthreads();
    const int gqa = a.Hq / a.Hkv > 0 ? a.Hq / a.Hkv : 1;
    const int total = a.B * a.Hq;
    for (int f = tid; f < total; f += blockDim.x) {
        if (a.flags[f] != 0) {
            const int hkv = (f % a.Hq) / gqa;
            if (hkv < a.Hkv) atomicMin(&first[hkv], f);
        }
    }
    __syncthreads();
    const int step = a.step_dev ? *a.step_dev : a.step;
    const int K = a.spike_k;
    if constexpr (TOPK) {
        __shared__ int allow_s[kMaxDrainHeads];  // tokens the head may queue, 0: not reached
        __shared__ uint8_t tok_kind[kMaxDrainHeads][FKV_MAX_SPIKE_K];
        __shared__ int tok_pos[kMaxDrainHeads][FKV_MAX_SPIKE_K], tok_arc[kMaxDrainHeads][FKV_MAX_SPIKE_K];
        for (int i = tid; i < kMaxDrainHeads; i += blockDim.x) allow_s[i] = 0;
        // every (KV head, token) outcome of the heads' first spikes, against the
        // state before this drain (a position repeated in a list: below)
        for (int u = tid; u < a.Hkv * K; u += blockDim.x) {
            const int h = u / K, j = u % K, f = first[h];
            int kind = kTokSkip, pos = 0, arc = -1;
            if (f != INT_MAX) {
                const int32_t last = a.last_step[h];
                const bool cooled = last != kNoStep && step - last < a.cooldown;
                const int n_tok = K > 1 ? (a.flags[f] < K ? a.flags[f] : K) : 1;
                if (!cooled && j < n_tok) {
                    uint32_t bit = 0;
                    int64_t widx = 0;
                    kind = drain_token(a, f, h, j, pos, arc, bit, widx);
                }
            }
            tok_kind[h][j] = (uint8_t)kind;
            tok_pos[h][j] = pos;
            tok_arc[h][j] = arc;
        }
        __syncthreads();
        // a position repeated in one head's list: the scan marks it at its first
        // occurrence, so every later occurrence is a duplicate (spike lists of
        // the attention kernel never repeat a token; other callers' may)
        // (the loops over a head's tokens run over all FKV_MAX_SPIKE_K entries
        // with the bound as a mask: their LDS reads issue together)
        if (K > 1) {
            uint32_t dup_bits = 0;  // bit n: this thread's n-th (KV head, token); at most 32 of them
            int n_mine = 0;
            for (int u = tid; u < a.Hkv * K; u += blockDim.x, n_mine++) {
                const int h = u / K, j = u % K, kind = tok_kind[h][j];
                if (kind == kTokMarked || kind == kTokQueued) {
                    const int pj = tok_pos[h][j];
                    bool dup = false;
#pragma unroll
                    for (int i = 0; i < FKV_MAX_SPIKE_K; i++) {
                        const int ki = tok_kind[h][i], pi = tok_pos[h][i];
                        dup |= (i < j) & (ki != kTokSkip) & (pi == pj);
                    }
                    if (dup) dup_bits |= 1u << n_mine;
                }
            }
            __syncthreads();
            n_mine = 0;
            for (int u = tid; u < a.Hkv * K; u += blockDim.x, n_mine++)
                if ((dup_bits >> n_mine) & 1u) tok_kind[u / K][u % K] = kTokDup;
            __syncthreads();
        }
        for (int h = tid; h < a.Hkv; h += blockDim.x) {
            int q = 0;
#pragma unroll
            for (int j = 0; j < FKV_MAX_SPIKE_K; j++) {
                const int kj = tok_kind[h][j];
                q += (j < K) & (kj == kTokQueued);
            }
            nq[h] = q;
        }
        __syncthreads();
        // thread h: KV head h's place in the scan, cooldown and counts
        for (int h = tid; h < a.Hkv; h += blockDim.x) {
            const int f = first[h];
            if (f == INT_MAX) continue;
            int before = 0;  // tokens the heads earlier in scan order queue
            for (int g = 0; g < a.Hkv; g++) before += first[g] < f ? nq[g] : 0;
            if (before >= a.budget) continue;
            atomicAdd(&cnt[0], 1u);
            const int32_t last = a.last_step[h];
            if (last != kNoStep && step - last < a.cooldown) {
                atomicAdd(&cnt[3], 1u);
                continue;
            }
            a.last_step[h] = step;
            const int allow = a.budget - before;
            const int cur = (int)((const uint32_t*)(a.blob + a.L.near_valid))[h];
            const int queued = nq[h] < allow ? nq[h] : allow;
            const int room = a.L.Na - cur > 0 ? a.L.Na - cur : 0;
            const int recs = queued < room ? queued : room;
            allow_s[h] = allow;
            n_rec[h] = recs;
            slot0[h] = cur;
            atomicAdd(&cnt[1], (unsigned)queued);
            atomicAdd(&cnt[4], (unsigned)recs);
            atomicAdd(&cnt[5], (unsigned)(queued - recs));
        }
        __syncthreads();
        // the tokens the scan reaches: fewer than `allow` queued tokens before them
        for (int u = tid; u < a.Hkv * K; u += blockDim.x) {
            const int h = u / K, j = u % K, allow = allow_s[h];
            const int kind = tok_kind[h][j];
            if (allow == 0 || kind == kTokSkip) continue;
            int qb = 0;
#pragma unroll
            for (int i = 0; i < FKV_MAX_SPIKE_K; i++) {
                const int ki = tok_kind[h][i];
                qb += (i < j) & (ki == kTokQueued);
            }
            if (qb >= allow) continue;
            if (kind == kTokDup) {
                atomicAdd(&cnt[2], 1u);
                continue;
            }
            const int pos = tok_pos[h][j];
            // tokens of one head may share a word of the bitmap
            atomicOr(a.promoted + (int64_t)h * a.words + (pos >> 5), 1u << (pos & 31));
            if (kind == kTokQueued && qb < n_rec[h]) rec_arc[h][qb] = tok_arc[h][j];
        }
    } else {
        // spike_k = 1: thread hkv scans its head's single token (the parallel
        // form above measured 0.8 us slower per call here)
        const int hkv = tid;
        const int f = hkv < a.Hkv ? first[hkv] : INT_MAX;
        bool cooled = false;
        int n_tok = 0;
        if (f != INT_MAX) {
            const int32_t last = a.last_step[hkv];
            cooled = last != kNoStep && step - last < a.cooldown;
            n_tok = K > 1 ? (a.flags[f] < K ? a.flags[f] : K) : 1;
            if (!cooled) {
                int q = 0;
                for (int j = 0; j < n_tok; j++) {
                    int pos = 0, arc = -1;
                    uint32_t bit = 0;
                    int64_t widx = 0;
                    q += drain_token(a, f, hkv, j, pos, arc, bit, widx) == kTokQueued;
                }
                nq[hkv] = q;
            }
        }
        __syncthreads();
        if (f != INT_MAX) {
            int before = 0;  // tokens the heads earlier in scan order queue
            for (int h = 0; h < a.Hkv; h++) before += first[h] < f ? nq[h] : 0;
            if (before < a.budget) {
                atomicAdd(&cnt[0], 1u);
                if (cooled) {
                    atomicAdd(&cnt[3], 1u);
                } else {
                    a.last_step[hkv] = step;
                    const int allow = a.budget - before;
                    const uint32_t cur = ((const uint32_t*)(a.blob + a.L.near_valid))[hkv];
                    int queued = 0, recs = 0;
                    unsigned dups = 0, full = 0;
                    for (int j = 0; j < n_tok && queued < allow; j++) {
                        int pos = 0, arc = -1;
                        uint32_t bit = 0;
                        int64_t widx = 0;
                        const int kind = drain_token(a, f, hkv, j, pos, arc, bit, widx);
                        if (kind == kTokSkip) continue;
                        if (kind == kTokDup) {
                            dups++;
                            continue;
                        }
                        a.promoted[widx] |= bit;
                        if (kind != kTokQueued) continue;
                        if ((int)cur + queued >= a.L.Na) full++;
                        else rec_arc[hkv][recs++] = arc;
                        queued++;
                    }
                    n_rec[hkv] = recs;
                    slot0[hkv] = (int)cur;
                    atomicAdd(&cnt[1], (unsigned)queued);
                    atomicAdd(&cnt[2], dups);
                    atomicAdd(&cnt[4], (unsigned)recs);
                    atomicAdd(&cnt[5], full);
                }
            }
        }
    }
    __syncthreads();
    if (tid < 6) a.stats[tid] += (unsigned long long)cnt[tid];
    const int nb = a.arc_B < a.L.B ? a.arc_B : a.L.B;
    uint16_t* nk = (uint16_t*)(a.blob + a.L.near_k);
    uint16_t* nv = (uint16_t*)(a.blob + a.L.near_v);
    // 16-byte reads of the archive (8 dims of a row: few, wide bus
    // transactions); the 8 K dims are contiguous in the near tile, the V
    // dims are 8 elements apart.  Every head's rows in one loop (item e:
    // record row r of all heads' records, batch, chunk), so the reads of
    // different heads are in flight together: roff[h] = the records of the
    // heads before h.
    __shared__ int roff[kMaxDrainHeads + 1];
    if (tid < a.Hkv) {
        int sum = 0;
        for (int g = 0; g <= tid; g++) sum += n_rec[g];
        roff[tid + 1] = sum;
    }
    if (tid == 0) roff[0] = 0;
    __syncthreads();
    const int D = a.L.D, DC = D / 8;
    const int nrows = roff[a.Hkv];
    for (int e = tid; e < nrows * nb * DC; e += blockDim.x) {
        const int c = e % DC, b = (e / DC) % nb, r = e / (DC * nb);
        int h = 0, hi = a.Hkv - 1;  // the last head with roff[h] <= r: the head of row r
        while (h < hi) {
            const int mid = (h + hi + 1) >> 1;
            if (roff[mid] <= r) h = mid;
            else hi = mid - 1;
        }
        const int i = r - roff[h];
        const int slot = slot0[h] + i;
        const int64_t base = ((int64_t)b * a.L.Hkv + h) * a.L.Na_pad * D;
        const int64_t src = (((int64_t)b * a.Hkv + h) * a.arc_S + rec_arc[h][i]) * D + 8 * c;
        const uint4 kw = *(const uint4*)(a.ark + src);
        const uint4 vw = *(const uint4*)(a.arv + src);
        *(uint4*)(nk + base + fkv::near_k_index(slot, 8 * c, D)) = kw;
        const uint32_t vv[4] = {vw.x, vw.y, vw.z, vw.w};
#pragma unroll
        for (int k = 0; k < 8; k++)
            nv[base + fkv::near_v_index(slot, 8 * c + k, D)] = (uint16_t)(vv[k >> 1] >> (16 * (k & 1)));
    }
    __syncthreads();
    for (int h = tid; h < a.Hkv; h += blockDim.x)
        if (n_rec[h] > 0) ((uint32_t*)(a.blob + a.L.near_valid))[h] = (uint32_t)(slot0[h] + n_rec[h]);
    // every thread read the step before the barriers above
    if (a.advance && tid == 0) *a.step_dev = step + 1;
}

// The step advance of a drain that has nothing to launch.
__global__ __launch_bounds__(64) void advance_step_kernel(int32_t* step_dev) {
    if (threadIdx.x == 0) *step_dev += 1;
}

// Device state of a layer for the device drain, made on its first use.
int ensure_dev_drain(fkv_promoter* p, int layer, hipStream_t st) {
    if (p->dev.empty()) p->dev.resize(p->n_layers);
    if (!p->dstats) {
        if (int rc = check_hip(hipMalloc((void**)&p->dstats, 6 * sizeof(unsigned long long)), "hipMalloc(stats)"))
            return rc;
        const unsigned long long zero[6] = {0, 0, 0, 0, 0, 0};
        if (int rc = check_hip(hipMemcpy(p->dstats, zero, sizeof(zero), hipMemcpyHostToDevice), "hipMemcpy(stats)"))
            return rc;
    }
    DevDrain& d = p->dev[layer];
    if (d.last_step) return FKV_OK;
    const Archive& a = p->arch[layer];
    if (!a.device && (!a.owned_k || !a.owned_v))
        return set_error("fkv_promoter_drain_device: the layer's archive is neither in pipeline-owned pinned memory "
                         "nor in device memory");
    int maxpos = -1;
    for (const auto& m : a.pos_to_local)
        for (const auto& kv : m) maxpos = kv.first > maxpos ? kv.first : maxpos;
    d.P = maxpos + 1;
    d.words = (d.P + 31) / 32;
    std::vector<int32_t> p2l((size_t)a.Hkv * (d.P > 0 ? d.P : 1), -1);
    for (int h = 0; h < a.Hkv; h++)
        for (const auto& kv : a.pos_to_local[h])
            if (kv.first >= 0) p2l[(size_t)h * d.P + kv.first] = kv.second;
    std::vector<int32_t> ls((size_t)a.Hkv, kNoStep);
    int rc = check_hip(hipMalloc((void**)&d.last_step, a.Hkv * sizeof(int32_t)), "hipMalloc(last_step)");
    if (!rc) rc = check_hip(hipMalloc((void**)&d.promoted, (size_t)a.Hkv * (d.words > 0 ? d.words : 1) * 4),
                            "hipMalloc(promoted)");
    if (!rc) rc = check_hip(hipMalloc((void**)&d.pos_to_local, p2l.size() * 4), "hipMalloc(pos_to_local)");
    if (!rc) rc = check_hip(hipMemcpy(d.last_step, ls.data(), ls.size() * 4, hipMemcpyHostToDevice), "hipMemcpy");
    if (!rc) rc = check_hip(hipMemset(d.promoted, 0, (size_t)a.Hkv * (d.words > 0 ? d.words : 1) * 4), "hipMemset");
    if (!rc) rc = check_hip(hipMemcpy(d.pos_to_local, p2l.data(), p2l.size() * 4, hipMemcpyHostToDevice), "hipMemcpy");
    void* dk = (void*)a.k;  // a device archive is read in place
    void* dv = (void*)a.v;
    if (!rc && !a.device) rc = check_hip(hipHostGetDevicePointer(&dk, a.owned_k, 0), "hipHostGetDevicePointer");
    if (!rc && !a.device) rc = check_hip(hipHostGetDevicePointer(&dv, a.owned_v, 0), "hipHostGetDevicePointer");
    if (rc) {
        if (d.last_step) (void)hipFree(d.last_step);
        if (d.promoted) (void)hipFree(d.promoted);
        if (d.pos_to_local) (void)hipFree(d.pos_to_local);
        d = DevDrain();
        return rc;
    }
    d.ark = (const uint16_t*)dk;
    d.arv = (const uint16_t*)dv;
    return FKV_OK;
}

}  // namespace

extern "C" {

int fkv_promoter_create(int32_t n_layers, int32_t cooldown_steps, int32_t max_per_drain, fkv_promoter** out) {
    if (!out) return set_error("fkv_promoter_create: out is NULL");
    *out = nullptr;
    if (n_layers <= 0 || n_layers > 65535 || max_per_drain < 0)
        return set_error("fkv_promoter_create: need 0 < n_layers <= 65535 and max_per_drain >= 0");
    fkv_promoter* p = new fkv_promoter();
    p->n_layers = n_layers;
    p->cooldown = cooldown_steps;
    p->max_per_drain = max_per_drain;
    p->arch.resize(n_layers);
    p->handles.assign(n_layers, nullptr);
    p->mirror.assign(n_layers, {});
    p->mode.assign(n_layers, kDrainNone);
    p->n_alloc.assign(n_layers, 0);
    *out = p;
    return FKV_OK;
}

int fkv_promoter_register_archive(fkv_promoter* p, int32_t layer, const void* k, const void* v, int32_t B,
                                  int32_t Hkv, int32_t S_arc, int32_t D, const int32_t* archive_idx,
                                  int32_t copy_to_pinned) {
    if (!p) return set_error("fkv_promoter_register_archive: NULL pipeline");
    if (layer < 0 || layer >= p->n_layers) return set_error("fkv_promoter_register_archive: layer out of range");
    if (B <= 0 || Hkv <= 0 || S_arc < 0 || D <= 0 || (S_arc > 0 && (!k || !v)))
        return set_error("fkv_promoter_register_archive: bad shape or NULL rows");
    Archive a;
    a.B = B;
    a.Hkv = Hkv;
    a.S = S_arc;
    a.D = D;
    const size_t bytes = (size_t)B * Hkv * S_arc * D * 2;
    if (copy_to_pinned && bytes) {
        int rc = check_hip(hipHostMalloc(&a.owned_k, bytes, hipHostMallocDefault), "hipHostMalloc(archive)");
        if (!rc) rc = check_hip(hipHostMalloc(&a.owned_v, bytes, hipHostMallocDefault), "hipHostMalloc(archive)");
        if (rc) {
            free_archive(a);
            return rc;
        }
        memcpy(a.owned_k, k, bytes);
        memcpy(a.owned_v, v, bytes);
        a.k = (const uint16_t*)a.owned_k;
        a.v = (const uint16_t*)a.owned_v;
    } else {
        a.k = (const uint16_t*)k;
        a.v = (const uint16_t*)v;
    }
    build_positions(a, archive_idx);
    free_dev_drain(p, layer);
    free_archive(p->arch[layer]);
    p->arch[layer] = std::move(a);
    return FKV_OK;
}

int fkv_promoter_register_archive_device(fkv_promoter* p, int32_t layer, const void* k, const void* v, int32_t B,
                                         int32_t Hkv, int32_t S_arc, int32_t D, const int32_t* archive_idx) {
    if (!p) return set_error("fkv_promoter_register_archive_device: NULL pipeline");
    if (layer < 0 || layer >= p->n_layers)
        return set_error("fkv_promoter_register_archive_device: layer out of range");
    if (B <= 0 || Hkv <= 0 || S_arc < 0 || D <= 0 || D % 8 != 0 || (S_arc > 0 && (!k || !v)))
        return set_error("fkv_promoter_register_archive_device: bad shape or NULL rows");
    hipPointerAttribute_t attr{};
    if (S_arc > 0 && (hipPointerGetAttributes(&attr, k) != hipSuccess || attr.type != hipMemoryTypeDevice ||
                      hipPointerGetAttributes(&attr, v) != hipSuccess || attr.type != hipMemoryTypeDevice)) {
        (void)hipGetLastError();
        return set_error("fkv_promoter_register_archive_device: the rows are not in device memory");
    }
    Archive a;
    a.B = B;
    a.Hkv = Hkv;
    a.S = S_arc;
    a.D = D;
    a.k = (const uint16_t*)k;
    a.v = (const uint16_t*)v;
    a.device = true;
    build_positions(a, archive_idx);
    free_dev_drain(p, layer);
    free_archive(p->arch[layer]);
    p->arch[layer] = std::move(a);
    return FKV_OK;
}

int fkv_promoter_register_archive_files(fkv_promoter* p, int32_t layer, const char* path_k, const char* path_v,
                                        int32_t Hkv, int32_t S_arc, int32_t D, const int32_t* archive_idx) {
    if (!p || !path_k || !path_v) return set_error("fkv_promoter_register_archive_files: NULL argument");
    if (layer < 0 || layer >= p->n_layers) return set_error("fkv_promoter_register_archive_files: layer out of range");
    if (Hkv <= 0 || S_arc < 0 || D <= 0) return set_error("fkv_promoter_register_archive_files: bad shape");
    const size_t bytes = (size_t)Hkv * S_arc * D * 2;
    Archive a;
    a.B = 1;
    a.Hkv = Hkv;
    a.S = S_arc;
    a.D = D;
    if (bytes) {
        int rc = check_hip(hipHostMalloc(&a.owned_k, bytes, hipHostMallocDefault), "hipHostMalloc(archive)");
        if (!rc) rc = check_hip(hipHostMalloc(&a.owned_v, bytes, hipHostMallocDefault), "hipHostMalloc(archive)");
        if (rc) {
            free_archive(a);
            return rc;
        }
        const char* paths[2] = {path_k, path_v};
        void* dst[2] = {a.owned_k, a.owned_v};
        for (int f = 0; f < 2; f++) {
            FILE* fp = fopen(paths[f], "rb");
            const size_t got = fp ? fread(dst[f], 1, bytes, fp) : 0;
            if (fp) fclose(fp);
            if (got != bytes) {  // the layer is left without an archive, as in the reference
                free_archive(a);
                free_dev_drain(p, layer);  // a queued device drain may still read the old rows
                free_archive(p->arch[layer]);
                return set_error(std::string("fkv_promoter_register_archive_files: cannot read ") +
                                 std::to_string(bytes) + " bytes from " + paths[f]);
            }
        }
        a.k = (const uint16_t*)a.owned_k;
        a.v = (const uint16_t*)a.owned_v;
    }
    build_positions(a, archive_idx);
    free_dev_drain(p, layer);
    free_archive(p->arch[layer]);
    p->arch[layer] = std::move(a);
    return FKV_OK;
}

int fkv_promoter_register_handle(fkv_promoter* p, int32_t layer, fkv_attn* h, void* stream) {
    if (!p || !h) return set_error("fkv_promoter_register_handle: NULL argument");
    if (layer < 0 || layer >= p->n_layers) return set_error("fkv_promoter_register_handle: layer out of range");
    fkv_blob_info bi;
    if (int rc = fkv_attn_blob_info(h, &bi)) return rc;
    std::vector<uint32_t> nv((size_t)bi.H_kv);
    if (int rc = fkv_attn_read_near_valid(h, nv.data(), stream)) return rc;
    p->handles[layer] = h;
    p->mirror[layer] = std::move(nv);
    p->mode[layer] = kDrainNone;  // a new blob: either drain may start on it
    p->n_alloc[layer] = bi.n_near_alloc;
    return FKV_OK;
}

// promotion_pipeline.cpp:99-175
int fkv_promoter_drain(fkv_promoter* p, int32_t layer, const int32_t* flags, const int32_t* tokens,
                       const int32_t* far_idx, int32_t B, int32_t Hq, int32_t Hkv, int32_t N_far, int32_t step) {
    if (!p) return set_error("fkv_promoter_drain: NULL pipeline");
    if (layer < 0 || layer >= p->n_layers) return 0;
    const Archive& a = p->arch[layer];
    if (!a.k || a.S == 0) return 0;  // no archive registered for the layer
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || !flags || !tokens || !far_idx) return 0;
    if (p->mode[layer] == kDrainDevice)
        return set_error("fkv_promoter_drain: layer " + std::to_string(layer) +
                         " is drained on the device; its headroom slots are assigned there");
    p->mode[layer] = kDrainHost;
    const int gqa = Hq / Hkv > 0 ? Hq / Hkv : 1;
    std::vector<uint8_t> seen((size_t)Hkv, 0);
    int queued = 0;
    for (int b = 0; b < B && queued < p->max_per_drain; b++) {
        for (int hq = 0; hq < Hq && queued < p->max_per_drain; hq++) {
            const int flat = b * Hq + hq;
            if (flags[flat] == 0) continue;
            const int hkv = hq / gqa;
            if (hkv >= Hkv || seen[hkv]) continue;
            seen[hkv] = 1;
            p->stats.spikes_detected++;
            const uint32_t cd_key = ((uint32_t)layer << 16) | (uint32_t)hkv;
            auto it = p->last_step.find(cd_key);
            if (it != p->last_step.end() && step - it->second < p->cooldown) {
                p->stats.spikes_cooled_down++;
                continue;
            }
            p->last_step[cd_key] = step;
            // the query head's spiking tokens (K > 1: flags holds their
            // count, tokens their far-local indices in descending score
            // order), each through the position dedup, the archive lookup
            // and the budget
            const int K = p->spike_k;
            const int n_tok = K > 1 ? (flags[flat] < K ? flags[flat] : K) : 1;
            for (int j = 0; j < n_tok && queued < p->max_per_drain; j++) {
                const int far_local = tokens[(int64_t)flat * K + j];
                if (far_local < 0 || far_local >= N_far) continue;
                const int32_t position = far_idx[((int64_t)b * Hkv + hkv) * N_far + far_local];
                const uint64_t key = ((uint64_t)(layer & 0xFFFF) << 48) | ((uint64_t)(hkv & 0xFFFF) << 32) |
                                     (uint64_t)(uint32_t)position;
                if (!p->promoted.insert(key).second) {
                    p->stats.spikes_deduplicated++;
                    continue;
                }
                if (hkv >= (int)a.pos_to_local.size()) continue;
                auto pit = a.pos_to_local[hkv].find(position);
                if (pit == a.pos_to_local[hkv].end()) continue;
                p->queue.push_back({layer, hkv, pit->second, position});
                p->stats.spikes_queued++;
                queued++;
            }
        }
    }
    return queued;
}

int fkv_promoter_set_spike_k(fkv_promoter* p, int32_t spike_k) {
    if (!p) return set_error("fkv_promoter_set_spike_k: NULL pipeline");
    if (spike_k < 1 || spike_k > FKV_MAX_SPIKE_K)
        return set_error("fkv_promoter_set_spike_k: spike_k must be in [1, " + std::to_string(FKV_MAX_SPIKE_K) +
                         "], got " + std::to_string(spike_k));
    p->spike_k = spike_k;
    return FKV_OK;
}

int fkv_promoter_pending(const fkv_promoter* p, int32_t* out_records, int32_t max_records) {
    if (!p) return set_error("fkv_promoter_pending: NULL pipeline");
    const int n = (int)p->queue.size();
    for (int i = 0; i < n && i < max_records && out_records; i++) {
        out_records[4 * i + 0] = p->queue[i].layer;
        out_records[4 * i + 1] = p->queue[i].head;
        out_records[4 * i + 2] = p->queue[i].arc_local;
        out_records[4 * i + 3] = p->queue[i].position;
    }
    return n;
}


int fkv_promoter_drain_device(fkv_promoter* p, int32_t layer, const int32_t* flags, const int32_t* tokens,
                              const int32_t* far_idx, int32_t B, int32_t Hq, int32_t Hkv, int32_t N_far, int32_t step,
                              int32_t* step_dev, int32_t advance_step, void* stream) {
    if (!p) return set_error("fkv_promoter_drain_device: NULL pipeline");
    if (advance_step && !step_dev) return set_error("fkv_promoter_drain_device: advance_step needs step_dev");
    hipStream_t st = (hipStream_t)stream;
    // a call with nothing to drain still advances the step
    auto nothing = [&]() -> int {
        if (!advance_step) return FKV_OK;
        hipLaunchKernelGGL(advance_step_kernel, dim3(1), dim3(64), 0, st, step_dev);
        return check_hip(hipGetLastError(), "advance_step_kernel launch");
    };
    if (layer < 0 || layer >= p->n_layers) return nothing();
    const Archive& arc = p->arch[layer];
    fkv_attn* h = p->handles[layer];
    if (!arc.k || arc.S == 0 || !h) return nothing();  // nothing to promote from or into (as the host drain)
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || !flags || !tokens || !far_idx) return nothing();
    if (Hkv > kMaxDrainHeads || Hkv != arc.Hkv || Hkv != h->L.Hkv || arc.D != h->L.D)
        return set_error("fkv_promoter_drain_device: archive, handle and spike shapes disagree (or H_kv > 256)");
    if (p->mode[layer] == kDrainHost)
        return set_error("fkv_promoter_drain_device: layer " + std::to_string(layer) +
                         " is drained on the host; its headroom slots are assigned there");
    p->mode[layer] = kDrainDevice;
    if (int rc = ensure_dev_drain(p, layer, st)) return rc;
    const DevDrain& d = p->dev[layer];
    DrainArgs a;
    a.flags = flags;
    a.tokens = tokens;
    a.far_idx = far_idx;
    a.B = B;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.N_far = N_far;
    a.step = step;
    a.step_dev = step_dev;
    a.advance = advance_step != 0;
    a.cooldown = p->cooldown;
    a.budget = p->max_per_drain;
    a.spike_k = p->spike_k;
    a.last_step = d.last_step;
    a.promoted = d.promoted;
    a.pos_to_local = d.pos_to_local;
    a.P = d.P;
    a.words = d.words;
    a.ark = d.ark;
    a.arv = d.arv;
    a.arc_B = arc.B;
    a.arc_S = arc.S;
    a.L = h->L;
    a.blob = h->blob;
    a.stats = p->dstats;
    if (p->spike_k > 1) hipLaunchKernelGGL(drain_promote_kernel<true>, dim3(1), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(drain_promote_kernel<false>, dim3(1), dim3(256), 0, st, a);
    return check_hip(hipGetLastError(), "drain_promote_kernel launch");
}

// promotion_pipeline.cpp:192-241, as stream-ordered device work
int fkv_promoter_flush(fkv_promoter* p) {
    if (!p) return set_error("fkv_promoter_flush: NULL pipeline");
    if (p->queue.empty()) return FKV_OK;
    if (int rc = ensure_gpu(p)) return rc;
    // assign headroom slots per layer from the mirrors; group by layer
    struct Item {
        int32_t head, slot, arc_local;
    };
    std::vector<std::vector<Item>> per(p->n_layers);
    for (const Record& r : p->queue) {
        fkv_attn* h = p->handles[r.layer];
        if (!h) continue;  // no blob registered: nothing to write into
        uint32_t& cur = p->mirror[r.layer][r.head];
        if ((int)cur >= p->n_alloc[r.layer]) {
            p->stats.promotions_headroom_full++;
            continue;
        }
        per[r.layer].push_back({r.head, (int32_t)cur, r.arc_local});
        cur++;
    }
    p->queue.clear();
    // staging: per layer [hs: 2n int32 | K rows: n*B*D fp16 | V rows: n*B*D fp16], 16-byte aligned
    size_t total = 0;
    std::vector<size_t> off(p->n_layers, 0);
    for (int l = 0; l < p->n_layers; l++) {
        if (per[l].empty()) continue;
        const Archive& a = p->arch[l];
        const size_t n = per[l].size();
        off[l] = total;
        total += align16(n * 8) + 2 * align16(n * (size_t)a.B * a.D * 2);
    }
    if (total == 0) return FKV_OK;
    if (int rc = ensure_staging(p, total)) return rc;
    if (p->staged_pending) {  // the previous copy out of the pinned staging has finished
        if (int rc = check_hip(hipEventSynchronize(p->staged), "hipEventSynchronize")) return rc;
        p->staged_pending = false;
    }
    for (int l = 0; l < p->n_layers; l++) {
        if (per[l].empty()) continue;
        const Archive& a = p->arch[l];
        const size_t n = per[l].size(), row = (size_t)a.D;
        int32_t* hs = (int32_t*)(p->stage_h + off[l]);
        uint16_t* rk = (uint16_t*)(p->stage_h + off[l] + align16(n * 8));
        uint16_t* rv = (uint16_t*)((uint8_t*)rk + align16(n * a.B * row * 2));
        for (size_t i = 0; i < n; i++) {
            const Item& it = per[l][i];
            hs[2 * i] = it.head;
            hs[2 * i + 1] = it.slot;
            if (a.device) continue;  // copied device to device below
            for (int b = 0; b < a.B; b++) {
                const size_t src = (((size_t)b * a.Hkv + it.head) * a.S + it.arc_local) * row;
                memcpy(rk + (i * a.B + b) * row, a.k + src, row * 2);
                memcpy(rv + (i * a.B + b) * row, a.v + src, row * 2);
            }
        }
    }
    int rc = check_hip(hipMemcpyAsync(p->stage_d, p->stage_h, total, hipMemcpyHostToDevice, p->side),
                       "hipMemcpyAsync(promotion rows)");
    // rows of device-resident archives: device-to-device into the device
    // staging, after (on the same stream) the copy of the host staging
    for (int l = 0; l < p->n_layers && !rc; l++) {
        const Archive& a = p->arch[l];
        if (per[l].empty() || !a.device) continue;
        const size_t n = per[l].size(), row = (size_t)a.D;
        uint16_t* rk = (uint16_t*)(p->stage_d + off[l] + align16(n * 8));
        uint16_t* rv = (uint16_t*)((uint8_t*)rk + align16(n * a.B * row * 2));
        for (size_t i = 0; i < n && !rc; i++)
            for (int b = 0; b < a.B && !rc; b++) {
                const size_t src = (((size_t)b * a.Hkv + per[l][i].head) * a.S + per[l][i].arc_local) * row;
                rc = check_hip(hipMemcpyAsync(rk + (i * a.B + b) * row, a.k + src, row * 2, hipMemcpyDeviceToDevice,
                                              p->side), "hipMemcpyAsync(device archive row)");
                if (!rc)
                    rc = check_hip(hipMemcpyAsync(rv + (i * a.B + b) * row, a.v + src, row * 2,
                                                  hipMemcpyDeviceToDevice, p->side),
                                   "hipMemcpyAsync(device archive row)");
            }
    }
    if (!rc) rc = check_hip(hipEventRecord(p->staged, p->side), "hipEventRecord");
    if (rc) return rc;
    p->staged_pending = true;
    for (int l = 0; l < p->n_layers && !rc; l++) {
        if (per[l].empty()) continue;
        const Archive& a = p->arch[l];
        const size_t n = per[l].size();
        const uint8_t* base = p->stage_d + off[l];
        const void* dk = base + align16(n * 8);
        const void* dv = (const uint8_t*)dk + align16(n * a.B * (size_t)a.D * 2);
        rc = fkv_attn_promote_rows(p->handles[l], (int32_t)n, (const int32_t*)base, dk, dv, a.B, p->side);
        if (!rc) rc = check_hip(hipEventRecord(p->done[l], p->side), "hipEventRecord");
        if (!rc) {
            p->has_done[l] = 1;
            p->stats.promotions_completed += n;
        }
    }
    return rc;
}

int fkv_promoter_order(fkv_promoter* p, int32_t layer, void* stream) {
    if (!p) return set_error("fkv_promoter_order: NULL pipeline");
    if (layer < 0 || layer >= p->n_layers || !p->side || !p->has_done[layer]) return FKV_OK;
    return check_hip(hipStreamWaitEvent((hipStream_t)stream, p->done[layer], 0), "hipStreamWaitEvent");
}

int fkv_promoter_synchronize(fkv_promoter* p) {
    if (!p) return set_error("fkv_promoter_synchronize: NULL pipeline");
    if (!p->side) return FKV_OK;
    return check_hip(hipStreamSynchronize(p->side), "hipStreamSynchronize");
}

int fkv_promoter_get_stats(const fkv_promoter* p, fkv_promoter_stats* out) {
    if (!p || !out) return set_error("fkv_promoter_get_stats: NULL argument");
    *out = p->stats;
    if (p->dstats) {  // device-drain counters (waits for the device)
        unsigned long long c[6];
        if (int rc = check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize")) return rc;
        if (int rc = check_hip(hipMemcpy(c, p->dstats, sizeof(c), hipMemcpyDeviceToHost), "hipMemcpy(stats)"))
            return rc;
        out->spikes_detected += c[0];
        out->spikes_queued += c[1];
        out->spikes_deduplicated += c[2];
        out->spikes_cooled_down += c[3];
        out->promotions_completed += c[4];
        out->promotions_headroom_full += c[5];
    }
    return FKV_OK;
}

int fkv_promoter_near_valid(const fkv_promoter* p, int32_t layer, uint32_t* out, int32_t n) {
    if (!p || !out) return set_error("fkv_promoter_near_valid: NULL argument");
    if (layer < 0 || layer >= p->n_layers) return set_error("fkv_promoter_near_valid: layer out of range");
    if (p->mode[layer] == kDrainDevice && p->handles[layer]) {
        // the device drain commits in the blob: read it there (after all queued work)
        fkv_attn* h = p->handles[layer];
        std::vector<uint32_t> nv((size_t)h->L.Hkv);
        if (int rc = check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize")) return rc;
        if (int rc = fkv_attn_read_near_valid(h, nv.data(), nullptr)) return rc;
        for (int i = 0; i < n && i < (int)nv.size(); i++) out[i] = nv[i];
        return (int)nv.size();
    }
    const auto& m = p->mirror[layer];
    for (int i = 0; i < n && i < (int)m.size(); i++) out[i] = m[i];
    return (int)m.size();
}

void fkv_promoter_destroy(fkv_promoter* p) {
    if (!p) return;
    if (p->side) {
        (void)hipStreamSynchronize(p->side);
        for (hipEvent_t e : p->done)
            if (e) (void)hipEventDestroy(e);
        if (p->staged) (void)hipEventDestroy(p->staged);
        (void)hipStreamDestroy(p->side);
    }
    if (p->stage_h) (void)hipHostFree(p->stage_h);
    if (p->stage_d) (void)hipFree(p->stage_d);
    if (p->dstats || !p->dev.empty()) (void)hipDeviceSynchronize();  // device drains may still run
    for (auto& d : p->dev) {
        if (d.last_step) (void)hipFree(d.last_step);
        if (d.promoted) (void)hipFree(d.promoted);
        if (d.pos_to_local) (void)hipFree(d.pos_to_local);
    }
    if (p->dstats) (void)hipFree(p->dstats);
    for (auto& a : p->arch) free_archive(a);
    delete p;
}

}  // extern "C"
