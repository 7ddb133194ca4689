// Prefill host side: workspace layout and the launches behind gdn_prefill_launch
// (plan, prep, then one scan launch, or two over segment job tables).
#include "gdn_prefill.h"

#include <algorithm>
#include <cmath>

// ------------------------------------------------------------------------- host side
namespace {

constexpr int64_t kChunkH = 64;
constexpr int kZeroFillBlocks = 64;

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

int64_t max_chunks(int64_t T, int64_t N) { return (T + kChunkH - 1) / kChunkH + N; }

// Segments per sequence (the default variant only): when (sequence, v-head) pairs are too
// few to fill 256 CUs, the largest G <= gdn::kSegMaxG whose pass-A jobs N HV (2 G - 3)
// still fit one workgroup per CU; 1 means no segments (G = 2 would scan its halves one
// after the other). The planner picks each sequence's count up to G from its length.
int seg_count(int64_t T, int64_t N, int64_t HV)
{
    // (the job planner runs one sequence per lane in the self-planned prep kernel)
    if (T <= 0 || N <= 0 || N > gdn::kSelfPlanMax || N * HV * 3 > 256)
        return 1;
    int64_t G = 3;
    while (G < gdn::kSegMaxG && N * HV * (2 * (G + 1) - 3) <= 256)
        ++G;
    // No sequence has more than ceil(T / 64) chunks, and the planner cuts one of c chunks
    // into at most min(G, c / kSegMinChunks, G*(c)) segments, G* its closed-form optimum
    // (rising with c; +1 for the device's float rounding). Capacities sized for that count
    // are tight for a single sequence (1 x 1024 at 8 v-heads: 4 segments instead of 16),
    // and below 3 no sequence is cut at all: one whole-sequence scan.
    const int64_t cmax = (T + kChunkH - 1) / kChunkH;
    const double w = gdn::kSegFirstWeight, h = 0.5 * gdn::kSegChainChunks;
    const int64_t gs = (int64_t)(1.0 - w + std::sqrt(w * w + w + (double)cmax / h)) + 1;
    G = std::min({G, cmax / gdn::kSegMinChunks, gs});
    return G >= 3 ? (int)G : 1;
}

struct Layout {
    int64_t nc;
    int64_t header, chunk_tok0, chunk_len, seq_chunk0, seq_rank, seq_tok0, seq_len, records,
        total;
    int G;                // segments per sequence at most (1: none)
    int64_t capA, capC;   // pass A / pass C job capacity
    int64_t jobs, seg_sin, seg_r, seg_mt;
};

Layout layout(int64_t T, int64_t N, int64_t HV)
{
    Layout L;
    L.G = seg_count(T, N, HV);
    L.capA = N * (2 * L.G - 3);
    L.capC = N * (L.G - 1);
    L.nc = max_chunks(T, N);
    int64_t o = 0;
    L.header = o;
    o += 64 * 4;
    L.chunk_tok0 = o;
    o += L.nc * 4;
    L.chunk_len = o;
    o += L.nc * 4;
    L.seq_chunk0 = o;
    o += (N + 1) * 4;
    L.seq_rank = (o + 15) & ~int64_t(15);
    o = L.seq_rank + N * 16;
    L.seq_tok0 = o;
    o += N * 4;
    L.seq_len = o;
    o += N * 4;
    L.records = align256(o);
    o = L.records + L.nc * HV * gdn::kRecBytes;
    L.jobs = L.seg_sin = L.seg_r = L.seg_mt = 0;
    if (L.G > 1) {
        const int64_t slot_bytes = N * (L.G - 1) * HV * gdn::kSlotFloats * 4;
        L.jobs = align256(o);
        o = L.jobs + (L.capA + L.capC) * gdn::kJobInts * 4;
        L.seg_sin = align256(o);
        L.seg_r = L.seg_sin + slot_bytes;
        L.seg_mt = L.seg_r + slot_bytes;
        o = L.seg_mt + slot_bytes;
    }
    L.total = o;
    return L;
}

bool aligned(const void *p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

// Compute units of the device that owns the stream (the current device when the
// stream is the null stream); 256 if the runtime cannot tell.
int num_cus(hipStream_t st)
{
    int dev = -1;
    if (st == nullptr || hipStreamGetDevice(st, &dev) != hipSuccess)
        if (hipGetDevice(&dev) != hipSuccess)
            return 256;
    static int cached[64] = {0};
    if (dev < 0 || dev >= 64)
        return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace

extern "C" int64_t gdn_prefill_workspace_size(int32_t total_tokens, int32_t num_seqs,
                                              int32_t num_qk_heads, int32_t num_v_heads,
                                              int32_t head_size)
{
    gdn_begin_call();
    if (total_tokens < 0 || num_seqs < 0 || num_qk_heads <= 0 || num_v_heads <= 0 ||
        num_v_heads % num_qk_heads != 0 || head_size != 128)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill_workspace_size: bad sizes T=%d N=%d "
                             "HQK=%d HV=%d D=%d", total_tokens, num_seqs, num_qk_heads,
                             num_v_heads, head_size);
    return layout(total_tokens, num_seqs, num_v_heads).total;
}

extern "C" int gdn_prefill_launch(const gdn_prefill_params *p, void *stream)
{
    gdn_begin_call();
    if (!p || p->struct_size != (int32_t)sizeof(gdn_prefill_params))
        return gdn_set_error(GDN_EINVAL, "gdn_prefill: params NULL or struct_size mismatch");
    const int T = p->total_tokens, N = p->num_seqs, HQK = p->num_qk_heads,
              HV = p->num_v_heads, D = p->head_size;
    if (T < 0 || N < 0 || HQK <= 0 || HV <= 0 || HV % HQK != 0)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill: bad sizes T=%d N=%d HQK=%d HV=%d", T, N,
                             HQK, HV);
    if (D != 128)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill: head_size %d unsupported (128 only)", D);
    if (p->variant < 0 || p->variant > 2)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill: variant %d unknown (0, 1, 2)", p->variant);
    if (!p->q || !p->k || !p->v || !p->A_log || !p->a || !p->dt_bias || !p->b ||
        !p->cu_seqlens || !p->output || !p->new_state)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill: NULL tensor pointer");
    if (p->q_stride[2] != 1 || p->k_stride[2] != 1 || p->v_stride[2] != 1 ||
        p->output_stride[2] != 1 || p->new_state_stride[3] != 1 ||
        (p->state && p->state_stride[3] != 1))
        return gdn_set_error(GDN_ELAYOUT, "gdn_prefill: innermost stride must be 1");
    for (int i = 0; i < 2; ++i)
        if (p->q_stride[i] % 8 || p->k_stride[i] % 8 || p->output_stride[i] % 8)
            return gdn_set_error(GDN_ELAYOUT,
                                 "gdn_prefill: q/k/output strides must be multiples of 8");
    for (int i = 0; i < 2; ++i)
        if (p->v_stride[i] % 8)
            return gdn_set_error(GDN_ELAYOUT, "gdn_prefill: v strides must be multiples of 8");
    if (!aligned(p->q, 16) || !aligned(p->k, 16) || !aligned(p->v, 16) || !aligned(p->output, 16))
        return gdn_set_error(GDN_ELAYOUT, "gdn_prefill: q/k/v/output must be 16-byte aligned");
    for (int i = 0; i < 3; ++i)
        if (p->new_state_stride[i] % 4 || (p->state && p->state_stride[i] % 4))
            return gdn_set_error(GDN_ELAYOUT,
                                 "gdn_prefill: state strides must be multiples of 4");
    if (!aligned(p->new_state, 16) || (p->state && !aligned(p->state, 16)))
        return gdn_set_error(GDN_ELAYOUT, "gdn_prefill: state must be 16-byte aligned");
    // the kernels address a 64-token chunk with 32-bit byte offsets
    const int64_t kMaxStride = int64_t(1) << 24;
    for (int i = 0; i < 2; ++i)
        if (p->q_stride[i] >= kMaxStride || p->k_stride[i] >= kMaxStride ||
            p->v_stride[i] >= kMaxStride || p->output_stride[i] >= kMaxStride ||
            p->q_stride[i] < 0 || p->k_stride[i] < 0 || p->v_stride[i] < 0 ||
            p->output_stride[i] < 0)
            return gdn_set_error(GDN_ELAYOUT,
                                 "gdn_prefill: token / head strides must be in [0, 2^24)");
    const int64_t kMaxGateStride = int64_t(1) << 31;
    for (int i = 0; i < 2; ++i)
        if (p->a_stride[i] < 0 || p->a_stride[i] >= kMaxGateStride || p->b_stride[i] < 0 ||
            p->b_stride[i] >= kMaxGateStride)
            return gdn_set_error(GDN_ELAYOUT, "gdn_prefill: a / b strides must be in [0, 2^31)");
    if (p->A_log_stride < 0 || p->A_log_stride >= kMaxGateStride || p->dt_bias_stride < 0 ||
        p->dt_bias_stride >= kMaxGateStride)
        return gdn_set_error(GDN_ELAYOUT, "gdn_prefill: A_log / dt_bias strides must be in [0, 2^31)");
    const Layout L = layout(T, N, HV);
    if (L.nc > 0x7fffffff)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill: too many chunks");
    if (!p->workspace || p->workspace_bytes < L.total || !aligned(p->workspace, 256))
        return gdn_set_error(GDN_EWORKSPACE,
                             "gdn_prefill: workspace needs %lld bytes, 256-byte aligned "
                             "(got %lld at %p)", (long long)L.total,
                             (long long)p->workspace_bytes, p->workspace);
    if (p->state && (const void *)p->state == (const void *)p->new_state)
        for (int i = 0; i < 4; ++i)
            if (p->state_stride[i] != p->new_state_stride[i])
                return gdn_set_error(GDN_ELAYOUT,
                                     "gdn_prefill: in-place state needs identical strides");

    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)p->workspace;
    const int ratio = HV / HQK;
    const int HO = HV;  // max(HQK, HV) with HV a multiple of HQK

    gdn::PlanArgs pa;
    pa.cu = p->cu_seqlens;
    pa.cu64 = p->cu_seqlens_int64 ? 1 : 0;
    pa.N = N;
    pa.T = T;
    pa.HO = HO;
    pa.nc = (int)L.nc;
    pa.header = (int32_t *)(ws + L.header);
    pa.chunk_tok0 = (int32_t *)(ws + L.chunk_tok0);
    pa.chunk_len = (int32_t *)(ws + L.chunk_len);
    pa.seq_chunk0 = (int32_t *)(ws + L.seq_chunk0);
    pa.seq_rank = (int32_t *)(ws + L.seq_rank);
    pa.seq_tok0 = (int32_t *)(ws + L.seq_tok0);
    pa.seq_len = (int32_t *)(ws + L.seq_len);
    pa.out = (gdn::bf16_t *)p->output;
    pa.o_st = p->output_stride[0];
    pa.o_sh = p->output_stride[1];
    // segments only for the default variant (the tuning variants keep whole sequences)
    const int G = p->variant == 0 ? L.G : 1;
    // Whole sequences: 4 scan waves per workgroup (two workgroups per (sequence, v-head))
    // when there are at most 128 (sequence, v-head) pairs, else 8 (129 to 256 pairs: the
    // device picks, whole_dual below). Variants: 1 forces 4 waves, 2 forces 8.
    const bool nw4 = p->variant == 1 || (p->variant == 0 && (int64_t)N * HV <= 128);
    pa.seg_G = G;
    pa.seg_capA = (int)L.capA;
    // Pass C: the 4-wave kernel (two workgroups per (job, v-head), spread over twice the CUs)
    // when its job capacity fits 128 pairs; otherwise both kernels are launched and the
    // planner gives the jobs to the 4-wave one whenever the plan's pass C fits 128 pairs
    // (every plan that cuts nothing, for one), else to the 8-wave one.
    const bool c4_only = L.capC * HV <= 128;
    pa.seg_c4 = G > 1 && !c4_only ? (int)(128 / HV) : 0;
    pa.jobs = G > 1 ? (int32_t *)(ws + L.jobs) : nullptr;
    // Up to 64 sequences the prep kernel plans for itself (one dependent launch fewer:
    // the plan kernel's ~5 us sat on the critical path, mostly cu_seqlens load latency).
    const bool prep_runs = L.nc > 0 && T > 0;
    const bool self_plan = prep_runs && N >= 1 && N <= gdn::kSelfPlanMax;
    // Whole sequences, 129 to 256 (sequence, v-head) pairs: either scan can be the faster,
    // depending on the longest sequence, which only the device knows. Both are launched
    // and the self-planning prep kernel gives the sequences to one of them; the other
    // launch finds none (~1.5-2 us for its up to 512 workgroups, one per CU at a time for
    // their LDS). Above 256 pairs the 8-wave scan alone (the 4-wave one rarely wins there).
    const bool whole_dual = G == 1 && p->variant == 0 && self_plan && (int64_t)N * HV > 128 &&
                            (int64_t)N * HV <= 256;
    pa.whole_cus = whole_dual ? num_cus(st) : 0;
    gdn_begin_launches();
    int rc = 0;
    if (!self_plan) {
        hipLaunchKernelGGL(gdn::gdn_prefill_plan_kernel, dim3(1 + kZeroFillBlocks), dim3(256),
                           0, st, pa);
        rc = gdn_check_launch("gdn_prefill_plan_kernel");
        if (rc)
            return rc;
    }

    if (prep_runs) {
        gdn::PrepArgs qa;
        qa.q = (const gdn::bf16_t *)p->q;
        qa.k = (const gdn::bf16_t *)p->k;
        qa.a = (const gdn::bf16_t *)p->a;
        qa.b = (const gdn::bf16_t *)p->b;
        qa.A_log = p->A_log;
        qa.dt_bias = p->dt_bias;
        qa.q_st = (int32_t)p->q_stride[0];
        qa.q_sh = (int32_t)p->q_stride[1];
        qa.k_st = (int32_t)p->k_stride[0];
        qa.k_sh = (int32_t)p->k_stride[1];
        qa.a_st = (int32_t)p->a_stride[0];
        qa.a_sh = (int32_t)p->a_stride[1];
        qa.b_st = (int32_t)p->b_stride[0];
        qa.b_sh = (int32_t)p->b_stride[1];
        qa.A_log_s = (int32_t)p->A_log_stride;
        qa.dt_s = (int32_t)p->dt_bias_stride;
        qa.header = pa.header;
        qa.chunk_tok0 = pa.chunk_tok0;
        qa.chunk_len = pa.chunk_len;
        qa.records = ws + L.records;
        qa.HQK = HQK;
        qa.HV = HV;
        qa.ratio = ratio;
        qa.scale = p->scale;
        qa.self_plan = self_plan ? 1 : 0;
        qa.plan = pa;
        // persistent: two workgroups per CU walk the (chunk, q/k head, v-head pair) units
        const int vh = ratio % 2 == 0 ? 2 : 1;
        const int64_t units = L.nc * HQK * (ratio / vh);
        const int64_t blocks = std::min<int64_t>(units, 2 * (int64_t)num_cus(st));
        if (blocks > 0x7fffffff)
            return gdn_set_error(GDN_EINVAL, "gdn_prefill: grid too large");
        if (vh == 2)
            hipLaunchKernelGGL(gdn::gdn_prefill_prep2_kernel, dim3((unsigned)blocks), dim3(512), 0,
                               st, qa);
        else
            hipLaunchKernelGGL(gdn::gdn_prefill_prep1_kernel, dim3((unsigned)blocks), dim3(256), 0,
                               st, qa);
        rc = gdn_check_launch("gdn_prefill_prep_kernel");
        if (rc)
            return rc;
    }

    if (N > 0) {
        gdn::ScanArgs sa;
        sa.q = (const gdn::bf16_t *)p->q;
        sa.k = (const gdn::bf16_t *)p->k;
        sa.v = (const gdn::bf16_t *)p->v;
        sa.state = p->state;
        sa.new_state = p->new_state;
        sa.out = (gdn::bf16_t *)p->output;
        sa.q_st = p->q_stride[0];
        sa.q_sh = p->q_stride[1];
        sa.k_st = p->k_stride[0];
        sa.k_sh = p->k_stride[1];
        sa.v_st = p->v_stride[0];
        sa.v_sh = p->v_stride[1];
        sa.o_st = p->output_stride[0];
        sa.o_sh = p->output_stride[1];
        sa.st_sn = p->state_stride[0];
        sa.st_sh = p->state_stride[1];
        sa.st_sv = p->state_stride[2];
        sa.ns_sn = p->new_state_stride[0];
        sa.ns_sh = p->new_state_stride[1];
        sa.ns_sv = p->new_state_stride[2];
        sa.header = pa.header;
        sa.seq_chunk0 = pa.seq_chunk0;
        sa.seq_rank = pa.seq_rank;
        sa.seq_tok0 = pa.seq_tok0;
        sa.seq_len = pa.seq_len;
        sa.records = ws + L.records;
        sa.HQK = HQK;
        sa.HV = HV;
        sa.ratio = ratio;
        sa.jobs = nullptr;
        sa.job_first = 0;
        sa.njob_idx = 0;
        sa.seg_sin = G > 1 ? (float *)(ws + L.seg_sin) : nullptr;
        sa.seg_r = G > 1 ? (float *)(ws + L.seg_r) : nullptr;
        sa.seg_mt = G > 1 ? (float *)(ws + L.seg_mt) : nullptr;
        // 8 waves per workgroup = one (sequence, v-head) each, two waves per SIMD; with
        // few (sequence, v-head) pairs, 4 waves and two workgroups per pair spread the
        // state rows over twice as many CUs. variant: 1 forces 4 waves, 2 forces 8.
        auto scan = [&](int64_t units, bool nw4) {
            const int64_t ngroups = units * HQK;
            sa.ngroups = (int)ngroups;
            const int tph = nw4 ? 2 : 1;
            const int64_t blocks = 8 * ((int64_t)tph * ratio) * ((ngroups + 7) / 8);
            if (ngroups > 0x7fffffff || blocks > 0x7fffffff)
                return gdn_set_error(GDN_EINVAL, "gdn_prefill: grid too large");
            const dim3 grid((unsigned)blocks), b4(256), b8(512);
            if (sa.jobs && nw4)
                hipLaunchKernelGGL(gdn::gdn_prefill_scan4_kernel<true>, grid, b4, 0, st, sa);
            else if (sa.jobs)
                hipLaunchKernelGGL(gdn::gdn_prefill_scan8_kernel<true>, grid, b8, 0, st, sa);
            else if (nw4)
                hipLaunchKernelGGL(gdn::gdn_prefill_scan4_kernel<false>, grid, b4, 0, st, sa);
            else
                hipLaunchKernelGGL(gdn::gdn_prefill_scan8_kernel<false>, grid, b8, 0, st, sa);
            return gdn_check_launch("gdn_prefill_scan_kernel");
        };
        if (G > 1) {
            // pass A: segment 0 of every sequence and both state maps of the middle segments
            sa.jobs = pa.jobs;
            sa.job_first = 0;
            sa.njob_idx = 1;
            rc = scan(L.capA, L.capA * HV <= 128);
            if (rc)
                return rc;
            // pass C: outputs of segments 1 .. G - 1, each chaining its entering state first;
            // the last segment's final state is new_state
            sa.job_first = (int)L.capA;
            sa.njob_idx = 2;
            rc = scan(c4_only ? L.capC : pa.seg_c4, true);
            if (rc == 0 && !c4_only) {
                sa.njob_idx = 3;
                rc = scan(L.capC, false);
            }
        } else if (whole_dual) {
            sa.njob_idx = 4;
            rc = scan(N, true);
            if (rc == 0) {
                sa.njob_idx = 5;
                rc = scan(N, false);
            }
        } else {
            rc = scan(N, nw4);
        }
        if (rc)
            return rc;
    }
    return GDN_OK;
}
