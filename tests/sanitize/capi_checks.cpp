// Host-side checks of the C ABI under AddressSanitizer and UndefinedBehaviorSanitizer: the
// config validation, the width / workspace / size queries and every entry point's argument
// checks, with valid, boundary and invalid inputs.  Built host-only (no device code) by
// `make -C hierarchicalglobalattention_amd/csrc sanitize`; calls that would reach a kernel
// launch are not made.  Exits non-zero on the first unexpected status; a sanitizer report
// aborts the run.
#include <hga.h>

#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>

static int g_fail = 0;

#define EXPECT(cond)                                                                      \
    do {                                                                                  \
        if (!(cond)) {                                                                    \
            std::fprintf(stderr, "%s:%d: expected %s (last error: %s)\n", __FILE__,       \
                         __LINE__, #cond, hga_last_error() ? hga_last_error() : "");      \
            ++g_fail;                                                                     \
        }                                                                                 \
    } while (0)

static hga_config base_cfg() {
    hga_config c;
    std::memset(&c, 0, sizeof(c));
    c.batch = 1;
    c.heads = 32;
    c.kv_heads = 4;
    c.head_dim = 128;
    c.chunk_size = 64;
    c.group_size = 16;
    c.topk_chunks = 16;
    c.topk_groups = 64;
    c.keep_first = 2;
    c.keep_last = 8;
    c.cutoff_pair = 20;
    c.dtype = HGA_DTYPE_BF16;
    c.scale = 0.08838835f;
    c.group_scale = 0.05f;
    return c;
}

static void config_checks() {
    int32_t N = 0, Kc = 0, Kg = 0;
    EXPECT(hga_prefill_widths(nullptr, 64, &N, &Kc, &Kg) == HGA_ERR_ARG);
    struct Bad {
        const char* what;
        void (*edit)(hga_config&);
        int code;
    } bad[] = {
        {"batch 0", [](hga_config& c) { c.batch = 0; }, HGA_ERR_ARG},
        {"heads % kv", [](hga_config& c) { c.heads = 30; }, HGA_ERR_ARG},
        {"kv 0", [](hga_config& c) { c.kv_heads = 0; }, HGA_ERR_ARG},
        {"head_dim 48", [](hga_config& c) { c.head_dim = 48; }, HGA_ERR_UNSUPPORTED},
        {"chunk 0", [](hga_config& c) { c.chunk_size = 0; }, HGA_ERR_UNSUPPORTED},
        {"chunk 65", [](hga_config& c) { c.chunk_size = 65; }, HGA_ERR_UNSUPPORTED},
        {"group 0", [](hga_config& c) { c.group_size = 0; }, HGA_ERR_ARG},
        {"group 24", [](hga_config& c) { c.group_size = 24; }, HGA_ERR_ARG},
        {"topk < 0", [](hga_config& c) { c.topk_chunks = -1; }, HGA_ERR_ARG},
        {"window < 0", [](hga_config& c) { c.keep_last = -3; }, HGA_ERR_ARG},
        {"cutoff", [](hga_config& c) { c.cutoff_pair = 65; }, HGA_ERR_ARG},
        {"dtype", [](hga_config& c) { c.dtype = 7; }, HGA_ERR_ARG},
        {"int max heads", [](hga_config& c) { c.heads = INT_MAX; c.kv_heads = 1; }, HGA_OK},
    };
    for (const Bad& b : bad) {
        hga_config c = base_cfg();
        b.edit(c);
        const int rc = hga_prefill_widths(&c, 4096, &N, &Kc, &Kg);
        if (rc != b.code) {
            std::fprintf(stderr, "config '%s': status %d, expected %d\n", b.what, rc, b.code);
            ++g_fail;
        }
    }
    hga_config c = base_cfg();
    EXPECT(hga_prefill_widths(&c, -1, &N, &Kc, &Kg) != HGA_OK);
    EXPECT(hga_prefill_widths(&c, 0, &N, &Kc, &Kg) == HGA_OK && N == 0);
    EXPECT(hga_prefill_widths(&c, INT_MAX, &N, &Kc, &Kg) == HGA_OK && N > 0 && Kc == 16);
    EXPECT(hga_decode_widths(&c, -1, &Kc, &Kg) != HGA_OK);
    EXPECT(hga_decode_widths(&c, 0, &Kc, &Kg) == HGA_OK && Kc == 0 && Kg == 0);
    EXPECT(hga_decode_widths(&c, INT_MAX / 64, &Kc, &Kg) == HGA_OK && Kc == 16 && Kg == 64);
    EXPECT(hga_version() > 0);
}

static void workspace_checks() {
    hga_config c = base_cfg();
    int64_t bytes = -1;
    EXPECT(hga_attend_prefill_workspace(&c, 32768, &bytes) == HGA_OK && bytes >= 0);
    EXPECT(hga_attend_prefill_workspace(&c, INT_MAX, &bytes) == HGA_OK && bytes > 0);
    EXPECT(hga_attend_prefill_workspace(&c, -5, &bytes) != HGA_OK);
    EXPECT(hga_attend_prefill_workspace(&c, 100, nullptr) != HGA_OK);
    EXPECT(hga_attend_prefill_bwd_workspace(&c, 32768, &bytes) == HGA_OK && bytes > 0);
    EXPECT(hga_attend_prefill_bwd_workspace(&c, INT_MAX, &bytes) == HGA_OK && bytes > 0);
    hga_config big = base_cfg();
    big.batch = 4096;
    big.heads = 1024;
    big.kv_heads = 512;
    EXPECT(hga_attend_prefill_bwd_workspace(&big, INT_MAX, &bytes) == HGA_OK && bytes > 0);
    for (int L : {1, 7, 64}) {
        EXPECT(hga_route_decode_workspace(&c, L, 0, &bytes) == HGA_OK && bytes >= 0);
        EXPECT(hga_route_decode_workspace(&c, L, 200000, &bytes) == HGA_OK && bytes > 0);
        // beyond (2048 / topk_chunks) segments of 2048 chunks
        EXPECT(hga_route_decode_workspace(&c, L, 1 << 20, &bytes) == HGA_ERR_UNSUPPORTED);
        EXPECT(hga_attend_decode_workspace(&c, L, 512, 512LL * 64, 64, &bytes) == HGA_OK);
    }
    EXPECT(hga_route_decode_workspace(&c, 0, 10, &bytes) != HGA_OK);
    EXPECT(hga_route_decode_workspace(&c, 65, 10, &bytes) != HGA_OK);
    EXPECT(hga_route_decode_workspace(&c, 1, -1, &bytes) != HGA_OK);
    EXPECT(hga_route_decode_workspace(&big, 64, INT_MAX / 64, &bytes) == HGA_ERR_UNSUPPORTED);
    EXPECT(hga_route_decode_workspace(&big, 64, 100000, &bytes) == HGA_OK && bytes > 0);
    EXPECT(hga_attend_decode_workspace(&c, 0, 10, 640, 8, &bytes) != HGA_OK);
    EXPECT(hga_attend_decode_workspace(&c, 1, 10, 640, -1, &bytes) != HGA_OK);
    EXPECT(hga_attend_decode_workspace(&big, 64, INT_MAX / 64, (int64_t)(INT_MAX / 64) * 64, 256,
                                       &bytes) == HGA_OK && bytes > 0);
    int32_t U = 0;
    int64_t sb = 0, xb = 0;
    EXPECT(hga_gather_decode_sizes(&c, 64, &U, &sb, &xb) == HGA_OK && U == 8 * 64 && sb > 0);
    EXPECT(hga_gather_decode_sizes(&c, -1, &U, &sb, &xb) != HGA_OK);
    EXPECT(hga_gather_decode_sizes(&big, INT_MAX / 4, &U, &sb, &xb) != HGA_OK ||
           (U > 0 && sb > 0));
}

// Entry points with arguments their checks refuse before any device call.
static void argument_checks() {
    hga_config c = base_cfg();
    char buf[256] __attribute__((aligned(16)));
    void* p = buf;
    int32_t* ip = reinterpret_cast<int32_t*>(buf);
    const float* fp = reinterpret_cast<const float*>(buf);
    EXPECT(hga_route_prefill(&c, 4096, nullptr, 0, 0, 0, p, 0, 0, p, 0, 0, ip, ip, ip, ip, ip,
                             ip, 0, nullptr, nullptr) == HGA_ERR_ARG);
    EXPECT(hga_route_prefill(&c, -1, p, 0, 0, 0, p, 0, 0, p, 0, 0, ip, ip, ip, ip, ip, ip, 0,
                             nullptr, nullptr) == HGA_ERR_ARG);
    EXPECT(hga_route_prefill(&c, 0, p, 0, 0, 0, p, 0, 0, p, 0, 0, ip, ip, ip, ip, ip, ip, 0,
                             nullptr, nullptr) == HGA_OK);
    // misaligned rows
    EXPECT(hga_route_prefill(&c, 4096, buf + 2, 0, 0, 128, p, 0, 0, p, 0, 0, ip, ip, ip, ip, ip,
                             ip, 0, nullptr, nullptr) == HGA_ERR_ARG);
    // pools beyond every routing kernel (fp32 takes 512 chunks)
    hga_config f = base_cfg();
    f.dtype = HGA_DTYPE_F32;
    EXPECT(hga_route_prefill(&f, 64 * 600, p, 0, 0, 128, p, 0, 128, p, 0, 512, ip, ip, ip, ip,
                             ip, ip, 0, nullptr, nullptr) == HGA_ERR_UNSUPPORTED);
    hga_config wide = base_cfg();
    wide.topk_chunks = 65;
    EXPECT(hga_route_prefill(&wide, 64 * 100, p, 0, 0, 128, p, 0, 128, p, 0, 512, ip, ip, ip, ip,
                             ip, ip, 0, nullptr, nullptr) == HGA_ERR_UNSUPPORTED);
    EXPECT(hga_attend_prefill(&c, 100, nullptr, 0, 0, 0, p, 0, 0, 0, p, 0, 0, 0, ip, ip, 64, p,
                              0, 0, 0, nullptr, p, 0, nullptr) != HGA_OK);
    EXPECT(hga_route_decode(&c, 0, 10, p, 0, 0, 0, p, 0, 0, p, 0, 0, ip, ip, ip, ip, ip, ip, p,
                            1 << 20, nullptr) != HGA_OK);
    EXPECT(hga_route_decode(&c, 1, 10, nullptr, 0, 0, 0, p, 0, 0, p, 0, 0, ip, ip, ip, ip, ip,
                            ip, p, 1 << 20, nullptr) != HGA_OK);
    // the block must lie inside the active chunk
    EXPECT(hga_attend_decode(&c, 4, 10, 10 * 64 + 62, p, 0, 0, 0, p, p, 0, 0, 0, 0, p, p, 0, 0,
                             0, p, p, 0, 0, 0, 0, ip, ip, 8, p, 0, 0, 0, p, 1 << 20,
                             nullptr) == HGA_ERR_ARG);
    EXPECT(hga_attend_decode(&c, 0, 10, 640, p, 0, 0, 0, p, p, 0, 0, 0, 0, p, p, 0, 0, 0, p, p,
                             0, 0, 0, 0, ip, ip, 8, p, 0, 0, 0, p, 1 << 20, nullptr) == HGA_ERR_ARG);
    EXPECT(hga_attend_decode_phase(&c, 1, 10, 640, p, 0, 0, 0, p, p, 0, 0, 0, 0, p, p, 0, 0, 0,
                                   p, p, 0, 0, 0, 0, ip, ip, 8, p, 0, 0, 0, 3, p, 1 << 20,
                                   nullptr) == HGA_ERR_ARG);
    // a workspace too small is refused before any launch
    EXPECT(hga_attend_decode(&c, 1, 10, 640, p, 0, 0, 0, p, p, 0, 0, 0, 0, p, p, 0, 0, 0, p, p,
                             0, 0, 0, 0, ip, ip, 8, p, 0, 0, 0, p, 16, nullptr) == HGA_ERR_ARG);
    // partials beyond the static scratch: refused before the device is touched
    hga_config b64 = base_cfg();
    b64.batch = 64;
    EXPECT(hga_attend_decode_noalloc(&b64, 64, 100, 6400, p, 0, 0, 0, p, p, 0, 0, 0, 0, p, p, 0,
                                     0, 0, p, p, 0, 0, 0, 0, ip, ip, 64, p, 0, 0, 0,
                                     nullptr) == HGA_ERR_UNSUPPORTED);
    EXPECT(hga_attend_decode_noalloc(&c, 0, 10, 640, p, 0, 0, 0, p, p, 0, 0, 0, 0, p, p, 0, 0, 0,
                                     p, p, 0, 0, 0, 0, ip, ip, 8, p, 0, 0, 0,
                                     nullptr) == HGA_ERR_ARG);
    EXPECT(hga_attend_decode_noalloc(&c, 1, 10, 700, nullptr, 0, 0, 0, p, p, 0, 0, 0, 0, p, p, 0,
                                     0, 0, p, p, 0, 0, 0, 0, ip, ip, 8, p, 0, 0, 0,
                                     nullptr) == HGA_ERR_ARG);
    EXPECT(hga_gather_decode(&c, 10, nullptr, ip, 8, p, p, 0, 0, 0, 0, p, p, 64, ip, p, 1 << 20,
                             nullptr) == HGA_ERR_ARG);
    EXPECT(hga_rope(&c, 4, 100, nullptr, 0, 0, 0, p, 0, 0, 0, fp, fp, 0, 0, nullptr) != HGA_OK);
}

int main() {
    config_checks();
    workspace_checks();
    argument_checks();
    if (g_fail) {
        std::fprintf(stderr, "capi_checks: %d failed\n", g_fail);
        return 1;
    }
    std::printf("capi_checks: ok\n");
    return 0;
}
