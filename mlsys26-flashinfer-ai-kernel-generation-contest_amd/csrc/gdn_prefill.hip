// Packed variable-length Gated DeltaNet prefill for gfx950 (chunked WY form).
#include "gdn_common.h"

namespace {
constexpr int64_t kChunk = 64;
constexpr int64_t kRecordBytes = 25600;  // per (chunk, v-head)

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

int64_t max_chunks(int64_t T, int64_t N) { return (T + kChunk - 1) / kChunk + N; }
}  // namespace

extern "C" int64_t gdn_prefill_workspace_size(int32_t total_tokens, int32_t num_seqs,
                                              int32_t num_qk_heads, int32_t num_v_heads,
                                              int32_t head_size)
{
    if (total_tokens < 0 || num_seqs < 0 || num_qk_heads <= 0 || num_v_heads <= 0 ||
        num_v_heads % num_qk_heads != 0 || head_size != 128)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill_workspace_size: bad sizes");
    const int64_t nc = max_chunks(total_tokens, num_seqs);
    const int64_t plan = align256(4 * (64 + 3 * nc + 4 * (int64_t(num_seqs) + 1)));
    return plan + nc * num_v_heads * kRecordBytes;
}

extern "C" int gdn_prefill_launch(const gdn_prefill_params *p, void *stream)
{
    (void)p; (void)stream;
    return gdn_set_error(GDN_EINVAL, "gdn_prefill: not built yet");
}
