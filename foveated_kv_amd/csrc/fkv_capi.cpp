// Library-wide C ABI entry points: errors, device probe, tier boundaries.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "fkv_common.h"
#include "../../include/fkv.h"

namespace fkv {

static thread_local std::string g_last_error;

int set_error(const std::string& msg) {
    g_last_error = msg;
    return FKV_EINVAL;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return FKV_OK;
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return e == hipErrorOutOfMemory ? FKV_ENOMEM : FKV_EHIP;
}

}  // namespace fkv

extern "C" {

const char* fkv_last_error(void) { return fkv::g_last_error.c_str(); }

int fkv_version(void) { return 200; }

int fkv_is_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) == hipSuccess && strncmp(p.gcnArchName, "gfx950", 6) == 0) return 1;
    }
    return 0;
}

// mlx_foveated.py:128-169 (Python int() truncation on double products)
int fkv_tier_boundaries(const fkv_tier_config* cfg, int32_t S, fkv_tiers* out) {
    if (!cfg || !out || S < 0) return fkv::set_error("fkv_tier_boundaries: bad argument");
    const int n_sinks = cfg->n_sinks < S ? cfg->n_sinks : S;
    const int rest = S - n_sinks > 0 ? S - n_sinks : 0;
    const int window = cfg->window_size < rest ? cfg->window_size : rest;
    const int reserved = n_sinks + window;
    int r_total = (int)((double)S * cfg->near_pct);
    if (r_total < reserved) r_total = reserved;
    if (S - r_total < 0) r_total = S;
    const int mid_start = n_sinks;
    const int mid_end = window > 0 ? S - window : S;
    const int mid_len = mid_end - mid_start > 0 ? mid_end - mid_start : 0;
    int from_mid = r_total - reserved > 0 ? r_total - reserved : 0;
    if (from_mid > mid_len) from_mid = mid_len;
    const int r_actual = n_sinks + from_mid + window;
    int headroom = (int)((double)r_actual * cfg->promo_headroom_pct);
    if (headroom < cfg->promo_headroom_min) headroom = cfg->promo_headroom_min;
    out->n_sinks = n_sinks;
    out->window = window;
    out->near_from_mid = from_mid;
    out->near_mid_start = mid_end - from_mid;
    out->far_count = out->near_mid_start - mid_start;
    out->r_actual = r_actual;
    out->headroom = headroom;
    out->n_near_padded = r_actual + headroom;
    out->mid_start = mid_start;
    out->mid_end = mid_end;
    return FKV_OK;
}

}  // extern "C"
