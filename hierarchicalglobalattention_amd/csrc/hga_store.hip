// Token ingest of a decode block (ChunkRouter.decode_block's store writes, chunk_router.py:279-300:
// the block's RoPE'd keys and values into the token record or ring, its raw keys into the
// active-chunk buffer the chunk's summaries are computed from when it closes).  One launch copies
// the three row sets; offsets are 64-bit, so a batched record far beyond 2^31 elements takes the
// same single launch.
#include "hga_common.h"

namespace hga {
namespace {

struct RowSet {
    const unsigned char* src;
    unsigned char* dst;
    int64_t s_sb, s_sh, s_ss, d_sb, d_sh, d_ss;   // byte strides (batch, head, row)
};

struct WriteArgs {
    RowSet set[3];
    int nset, B, X, L, V;   // V: 16-byte pieces per row
};

__global__ __launch_bounds__(256) void write_rows_kernel(WriteArgs A) {
    const int64_t per = (int64_t)A.B * A.X * A.L * A.V;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < per * A.nset;
         i += (int64_t)gridDim.x * blockDim.x) {
        const RowSet& R = A.set[i / per];
        int64_t r = i % per;
        const int v = (int)(r % A.V);
        r /= A.V;
        const int l = (int)(r % A.L);
        r /= A.L;
        const int x = (int)(r % A.X), b = (int)(r / A.X);
        const uint4 u = *reinterpret_cast<const uint4*>(R.src + b * R.s_sb + x * R.s_sh + l * R.s_ss +
                                                        16 * v);
        *reinterpret_cast<uint4*>(R.dst + b * R.d_sb + x * R.d_sh + l * R.d_ss + 16 * v) = u;
    }
}

}  // namespace
}  // namespace hga

extern "C" int hga_write_tokens(const hga_config* cfg, int32_t L, const void* k, int64_t k_sb,
                                int64_t k_sh, int64_t k_ss, const void* v, int64_t v_sb,
                                int64_t v_sh, int64_t v_ss, const void* k_raw, int64_t r_sb,
                                int64_t r_sh, int64_t r_ss, void* dst_k, int64_t dk_sb,
                                int64_t dk_sh, int64_t dk_ss, void* dst_v, int64_t dv_sb,
                                int64_t dv_sh, int64_t dv_ss, void* dst_raw, int64_t dr_sb,
                                int64_t dr_sh, int64_t dr_ss, void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(L >= 0, HGA_ERR_ARG, "hga_write_tokens: negative L");
    if (L == 0) return HGA_OK;
    const int64_t esz = cfg->dtype == HGA_DTYPE_BF16 ? 2 : 4;
    HGA_REQUIRE((cfg->head_dim * esz) % 16 == 0, HGA_ERR_UNSUPPORTED,
                "hga_write_tokens: rows of %lld bytes are not whole 16-byte pieces",
                (long long)(cfg->head_dim * esz));
    WriteArgs a{};
    const void* srcs[3] = {k, v, k_raw};
    void* dsts[3] = {dst_k, dst_v, dst_raw};
    const int64_t ss[3][3] = {{k_sb, k_sh, k_ss}, {v_sb, v_sh, v_ss}, {r_sb, r_sh, r_ss}};
    const int64_t ds[3][3] = {{dk_sb, dk_sh, dk_ss}, {dv_sb, dv_sh, dv_ss}, {dr_sb, dr_sh, dr_ss}};
    for (int s = 0; s < 3; ++s) {
        if (!srcs[s] && !dsts[s]) continue;   // a set may be left out with both pointers NULL
        HGA_REQUIRE(srcs[s] && dsts[s], HGA_ERR_ARG, "hga_write_tokens: row set %d half given", s);
        const uintptr_t al = (uintptr_t)srcs[s] | (uintptr_t)dsts[s];
        HGA_REQUIRE(al % 16 == 0 && ((ss[s][0] | ss[s][1] | ss[s][2] | ds[s][0] | ds[s][1] |
                                      ds[s][2]) * esz) % 16 == 0,
                    HGA_ERR_ARG, "hga_write_tokens: 16-byte aligned rows required");
        RowSet& R = a.set[a.nset++];
        R.src = static_cast<const unsigned char*>(srcs[s]);
        R.dst = static_cast<unsigned char*>(dsts[s]);
        R.s_sb = ss[s][0] * esz; R.s_sh = ss[s][1] * esz; R.s_ss = ss[s][2] * esz;
        R.d_sb = ds[s][0] * esz; R.d_sh = ds[s][1] * esz; R.d_ss = ds[s][2] * esz;
    }
    if (a.nset == 0) return HGA_OK;
    a.B = cfg->batch;
    a.X = cfg->kv_heads;
    a.L = L;
    a.V = (int)(cfg->head_dim * esz / 16);
    const int64_t total = (int64_t)a.nset * a.B * a.X * a.L * a.V;
    const unsigned grid = (unsigned)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    write_rows_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(a);
    return launch_status("hga_write_tokens");
}
