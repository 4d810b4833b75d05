// Host-side helpers of libhga: error reporting, config validation, small size queries.
#include <stdarg.h>
#include <stdio.h>

#include "hga_common.h"

namespace hga {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: %s", what, hipGetErrorString(e));
        return HGA_ERR_LAUNCH;
    }
    return HGA_OK;
}

int check_config(const hga_config* c) {
    HGA_REQUIRE(c != nullptr, HGA_ERR_ARG, "config is NULL");
    HGA_REQUIRE(c->batch > 0 && c->heads > 0 && c->kv_heads > 0, HGA_ERR_ARG,
                "batch/heads/kv_heads must be positive");
    HGA_REQUIRE(c->heads % c->kv_heads == 0, HGA_ERR_ARG, "heads (%d) %% kv_heads (%d) != 0",
                c->heads, c->kv_heads);
    HGA_REQUIRE(c->head_dim == 16 || c->head_dim == 32 || c->head_dim == 64 ||
                    c->head_dim == 128,
                HGA_ERR_UNSUPPORTED, "head_dim %d not in {16,32,64,128}", c->head_dim);
    HGA_REQUIRE(c->chunk_size > 0 && c->chunk_size <= 64, HGA_ERR_UNSUPPORTED,
                "chunk_size %d outside [1, 64]", c->chunk_size);
    HGA_REQUIRE(c->group_size > 0 && c->chunk_size % c->group_size == 0, HGA_ERR_ARG,
                "chunk_size %% group_size != 0");
    HGA_REQUIRE(c->topk_chunks >= 0 && c->topk_groups >= 0, HGA_ERR_ARG, "negative top-k");
    HGA_REQUIRE(c->keep_first >= 0 && c->keep_last >= 0, HGA_ERR_ARG, "negative window");
    HGA_REQUIRE(c->cutoff_pair >= 0 && c->cutoff_pair <= c->head_dim / 2, HGA_ERR_ARG,
                "cutoff_pair %d outside [0, head_dim/2]", c->cutoff_pair);
    HGA_REQUIRE(c->dtype == HGA_DTYPE_F32 || c->dtype == HGA_DTYPE_BF16, HGA_ERR_ARG,
                "unknown dtype %d", c->dtype);
    return HGA_OK;
}

}  // namespace hga

extern "C" int32_t hga_version(void) { return 100; }

extern "C" const char* hga_last_error(void) { return hga::g_err; }

extern "C" int32_t hga_prefill_widths(const hga_config* cfg, int32_t S, int32_t* N, int32_t* Kc,
                                      int32_t* Kg) {
    int rc = hga::check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(S >= 0, HGA_ERR_ARG, "negative S");
    const int n = hga::chunks_of(S, cfg->chunk_size);
    const int M = cfg->chunk_size / cfg->group_size;
    const int kc = cfg->topk_chunks > 0 ? (cfg->topk_chunks < n ? cfg->topk_chunks : n) : 0;
    const int kg = cfg->topk_groups > 0 ? (cfg->topk_groups < kc * M ? cfg->topk_groups : kc * M) : 0;
    if (N) *N = n;
    if (Kc) *Kc = kc;
    if (Kg) *Kg = kg;
    return HGA_OK;
}
