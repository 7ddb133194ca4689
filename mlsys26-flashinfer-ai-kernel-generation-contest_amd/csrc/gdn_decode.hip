// Single-token Gated DeltaNet decode for gfx950.
//
// Memory-bound: each (sequence, v-head) owns a 128 x 128 fp32 k-last state
// (64 KiB) that is read once and written once; everything else is < 1% of the
// bytes. One pass over the state computes both row dot products (S k and S q)
// from registers, so the update never re-reads HBM:
//   u = alpha (S k),  delta = beta v + (1 - beta) u - u
//   S' = alpha S + delta k^T,  o = scale (alpha (S q) + delta (k . q))
// which is the reference's per-row arithmetic
// (gdn_decode/solution/triton/kernel.py:120-131,165-170,216-218) with the readout
// S' q expanded so that it needs no second sweep over S'.
//
// seq_len T > 1 follows the reference kernel, whose programs (b, h, tile, t) each start
// from the input state (gdn_decode/solution/triton/kernel.py:117-118,146-147): token t's
// output is one decode step from the input state. The reference lets every token store
// new_state; here only token T - 1 stores it, so the result is deterministic.
//
// Thread mapping (default): a workgroup of 256 lanes covers 32 state rows; each
// row is spread over 8 consecutive lanes and each lane owns 16 columns as four
// float4 at columns 4s + 32j (s = lane % 8, j = 0..3), so one load instruction
// of a wavefront covers eight full 128-byte row segments. Row sums are 8-lane
// DPP reductions. Tuning variants change the workgroup size, lanes per row
// (8 or 16) and rows per lane.
#include "gdn_common.h"

namespace gdn {

struct DecodeArgs {
    const bf16_t *q, *k, *v;
    const float *state;
    const float *A_log;
    const bf16_t *a;
    const float *dt_bias;
    const bf16_t *b;
    bf16_t *out;
    float *new_state;
    int64_t q_sb, q_st, q_sh, k_sb, k_st, k_sh, v_sb, v_st, v_sh;
    int64_t st_sb, st_sh, st_sv;
    int64_t a_sb, a_st, a_sh, b_sb, b_st, b_sh;
    int64_t o_sb, o_st, o_sh;
    int64_t ns_sb, ns_sh, ns_sv;
    int64_t A_log_s, dt_s;
    int B, T, HV, ratio;
    float scale;
};

constexpr int kD = 128;

template <bool NT>
__device__ __forceinline__ f32x4 ld4(const float *p)
{
    if constexpr (NT)
        return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
    else
        return *reinterpret_cast<const f32x4 *>(p);
}

template <bool NT>
__device__ __forceinline__ void st4(float *p, f32x4 x)
{
    if constexpr (NT)
        __builtin_nontemporal_store(x, reinterpret_cast<f32x4 *>(p));
    else
        *reinterpret_cast<f32x4 *>(p) = x;
}

template <int LPR>
__device__ __forceinline__ float row_sum(float x)
{
    if constexpr (LPR == 8)
        return group8_sum(x);
    else
        return group16_sum(x);
}

// THREADS lanes per workgroup, LPR lanes per state row (8 or 16), RPT rows per lane.
// Lane s of a row owns the float4 column groups 4s + 4*LPR*j, j < NV4.
template <int THREADS, int LPR, int RPT, bool NT, bool HAS_STATE>
__global__ __launch_bounds__(THREADS) void gdn_decode_kernel(DecodeArgs p)
{
    constexpr int kRowsPerPass = THREADS / LPR;
    constexpr int kNV4 = kD / (4 * LPR);             // float4 per lane per row
    constexpr int kNVT = kD / (kRowsPerPass * RPT);  // workgroups per state
    constexpr int kCols = 4 * kNV4;                  // columns per lane
    const int bid = blockIdx.x;
    const int vt = bid % kNVT;
    const int bh = bid / kNVT;
    const int h = bh % p.HV;
    const int bt = bh / p.HV;
    const int bi = bt % p.B;
    const int t = bt / p.B;  // token; every token starts from the input state
    const int g = h / p.ratio;  // GVA: q/k head of this v-head (kernel.py:120)
    const int tid = threadIdx.x;
    const int s = tid % LPR;
    const int rg = tid / LPR;

    const int v0 = vt * kRowsPerPass * RPT;

    // Load order matters: vector loads return in issue order, so the few small loads
    // (gates, k, q, v) go first and the state stream right after; the gate math then
    // waits only for the small ones while the state is still in flight.
    const uint32_t a_raw = p.a[bi * p.a_sb + t * p.a_st + h * p.a_sh];
    const uint32_t b_raw = p.b[bi * p.b_sb + t * p.b_st + h * p.b_sh];
    u32x2 kraw[kNV4], qraw[kNV4];
    {
        const bf16_t *kp = p.k + bi * p.k_sb + t * p.k_st + g * p.k_sh + 4 * s;
        const bf16_t *qp = p.q + bi * p.q_sb + t * p.q_st + g * p.q_sh + 4 * s;
#pragma unroll
        for (int j = 0; j < kNV4; ++j) {
            kraw[j] = *reinterpret_cast<const u32x2 *>(kp + 4 * LPR * j);
            qraw[j] = *reinterpret_cast<const u32x2 *>(qp + 4 * LPR * j);
        }
    }
    uint32_t vraw[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r)
        vraw[r] = p.v[bi * p.v_sb + t * p.v_st + h * p.v_sh + v0 + rg + kRowsPerPass * r];
    __builtin_amdgcn_sched_barrier(0);

    f32x4 S[RPT][kNV4];
    if constexpr (HAS_STATE) {
        const float *sbase = p.state + bi * p.st_sb + h * p.st_sh;
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const float *row = sbase + (int64_t)(v0 + rg + kRowsPerPass * r) * p.st_sv + 4 * s;
#pragma unroll
            for (int j = 0; j < kNV4; ++j)
                S[r][j] = ld4<NT>(row + 4 * LPR * j);
        }
    }
    // the two scheduling barriers pin this issue order
    __builtin_amdgcn_sched_barrier(0);

    // Gates (gdn_decode/solution/triton/kernel.py:123-131), computed while the state
    // is in flight.
    const float A_log = p.A_log[h * p.A_log_s];
    const float dtb = p.dt_bias[h * p.dt_s];
    const float x = bf16_to_f32(a_raw) + dtb;
    const float sp = x > 20.f ? x : logf(1.f + expf(x));
    const float alpha = expf(-expf(A_log) * sp);
    const float beta = 1.f / (1.f + expf(-bf16_to_f32(b_raw)));

    float kk[kCols], qq[kCols];
#pragma unroll
    for (int j = 0; j < kNV4; ++j) {
        kk[4 * j + 0] = bf16lo(kraw[j].x);
        kk[4 * j + 1] = bf16hi(kraw[j].x);
        kk[4 * j + 2] = bf16lo(kraw[j].y);
        kk[4 * j + 3] = bf16hi(kraw[j].y);
        qq[4 * j + 0] = bf16lo(qraw[j].x);
        qq[4 * j + 1] = bf16hi(qraw[j].x);
        qq[4 * j + 2] = bf16lo(qraw[j].y);
        qq[4 * j + 3] = bf16hi(qraw[j].y);
    }
    float vrow[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r)
        vrow[r] = bf16_to_f32(vraw[r]);

    float kq = 0.f;
#pragma unroll
    for (int i = 0; i < kCols; ++i)
        kq = fmaf(kk[i], qq[i], kq);
    kq = row_sum<LPR>(kq);

    float *nbase = p.new_state + bi * p.ns_sb + h * p.ns_sh;
    bf16_t *obase = p.out + bi * p.o_sb + t * p.o_st + h * p.o_sh;
    const bool store_state = t == p.T - 1;
    const float omb = 1.f - beta;
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int row = v0 + rg + kRowsPerPass * r;
        float sk = 0.f, sq = 0.f;
        if constexpr (HAS_STATE) {
#pragma unroll
            for (int j = 0; j < kNV4; ++j) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sk = fmaf(S[r][j][e], kk[4 * j + e], sk);
                    sq = fmaf(S[r][j][e], qq[4 * j + e], sq);
                }
            }
            sk = row_sum<LPR>(sk);
            sq = row_sum<LPR>(sq);
        }
        const float u = alpha * sk;                  // (alpha S) k      kernel.py:165-166
        const float nv = beta * vrow[r] + omb * u;   // kernel.py:167
        const float d = nv - u;                      // kernel.py:168
        const float o = fmaf(alpha, sq, d * kq);     // (alpha S + d k^T) q
        float *nrow = nbase + (int64_t)row * p.ns_sv + 4 * s;
        if (store_state) {
#pragma unroll
            for (int j = 0; j < kNV4; ++j) {
                f32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float sv = HAS_STATE ? S[r][j][e] : 0.f;
                    w[e] = fmaf(alpha, sv, d * kk[4 * j + e]);  // kernel.py:169
                }
                st4<NT>(nrow + 4 * LPR * j, w);
            }
        }
        if (s == 0)
            obase[row] = (bf16_t)f32_to_bf16(p.scale * o);  // kernel.py:216-218
    }
}

}  // namespace gdn

namespace {

using gdn::DecodeArgs;

template <int THREADS, int LPR, int RPT, bool NT>
int launch_cfg(const DecodeArgs &a, int64_t nstates, hipStream_t stream)
{
    constexpr int kNVT = gdn::kD / ((THREADS / LPR) * RPT);
    const int64_t blocks = (int64_t)nstates * kNVT;
    if (blocks > 0x7fffffff)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: grid too large (%lld workgroups)",
                             (long long)blocks);
    if (a.state)
        hipLaunchKernelGGL((gdn::gdn_decode_kernel<THREADS, LPR, RPT, NT, true>),
                           dim3((unsigned)blocks), dim3(THREADS), 0, stream, a);
    else
        hipLaunchKernelGGL((gdn::gdn_decode_kernel<THREADS, LPR, RPT, NT, false>),
                           dim3((unsigned)blocks), dim3(THREADS), 0, stream, a);
    return gdn_check_launch("gdn_decode_kernel");
}

bool aligned(const void *p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

}  // namespace

extern "C" int gdn_decode_launch(const gdn_decode_params *p, void *stream)
{
    if (!p || p->struct_size != (int32_t)sizeof(gdn_decode_params))
        return gdn_set_error(GDN_EINVAL, "gdn_decode: params NULL or struct_size mismatch");
    const int B = p->batch, T = p->seq_len, HQK = p->num_qk_heads, HV = p->num_v_heads,
              D = p->head_size;
    if (B < 0 || HQK <= 0 || HV <= 0 || HV % HQK != 0)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: bad sizes B=%d HQK=%d HV=%d", B, HQK, HV);
    if (D != 128)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: head_size %d unsupported (128 only)", D);
    if (T < 1)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: seq_len %d must be >= 1", T);
    if (B == 0)
        return GDN_OK;
    if (!p->q || !p->k || !p->v || !p->A_log || !p->a || !p->dt_bias || !p->b || !p->output ||
        !p->new_state)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: NULL tensor pointer");
    if (p->q_stride[3] != 1 || p->k_stride[3] != 1 || p->v_stride[3] != 1 ||
        p->output_stride[3] != 1 || p->new_state_stride[3] != 1 ||
        (p->state && p->state_stride[3] != 1))
        return gdn_set_error(GDN_ELAYOUT, "gdn_decode: innermost stride must be 1");
    for (int i = 0; i < 3; ++i)
        if (p->q_stride[i] % 4 || p->k_stride[i] % 4)
            return gdn_set_error(GDN_ELAYOUT, "gdn_decode: q/k strides must be multiples of 4");
    if (!aligned(p->q, 8) || !aligned(p->k, 8))
        return gdn_set_error(GDN_ELAYOUT, "gdn_decode: q/k must be 8-byte aligned");
    for (int i = 0; i < 3; ++i)
        if (p->new_state_stride[i] % 4 || (p->state && p->state_stride[i] % 4))
            return gdn_set_error(GDN_ELAYOUT,
                                 "gdn_decode: state strides must be multiples of 4");
    if (!aligned(p->new_state, 16) || (p->state && !aligned(p->state, 16)))
        return gdn_set_error(GDN_ELAYOUT, "gdn_decode: state must be 16-byte aligned");
    if (p->state && (const void *)p->state != (const void *)p->new_state) {
        // Distinct buffers are fine; identical buffers must also share strides.
    } else if (p->state) {
        if (T > 1)
            return gdn_set_error(GDN_EINVAL, "gdn_decode: seq_len > 1 reads the input state "
                                 "for every token; new_state must not alias state");
        for (int i = 0; i < 4; ++i)
            if (p->state_stride[i] != p->new_state_stride[i])
                return gdn_set_error(GDN_ELAYOUT,
                                     "gdn_decode: in-place state needs identical strides");
    }

    DecodeArgs a;
    a.q = (const gdn::bf16_t *)p->q;
    a.k = (const gdn::bf16_t *)p->k;
    a.v = (const gdn::bf16_t *)p->v;
    a.state = p->state;
    a.A_log = p->A_log;
    a.a = (const gdn::bf16_t *)p->a;
    a.dt_bias = p->dt_bias;
    a.b = (const gdn::bf16_t *)p->b;
    a.out = (gdn::bf16_t *)p->output;
    a.new_state = p->new_state;
    a.q_sb = p->q_stride[0];
    a.q_st = p->q_stride[1];
    a.q_sh = p->q_stride[2];
    a.k_sb = p->k_stride[0];
    a.k_st = p->k_stride[1];
    a.k_sh = p->k_stride[2];
    a.v_sb = p->v_stride[0];
    a.v_st = p->v_stride[1];
    a.v_sh = p->v_stride[2];
    a.st_sb = p->state_stride[0];
    a.st_sh = p->state_stride[1];
    a.st_sv = p->state_stride[2];
    a.a_sb = p->a_stride[0];
    a.a_st = p->a_stride[1];
    a.a_sh = p->a_stride[2];
    a.b_sb = p->b_stride[0];
    a.b_st = p->b_stride[1];
    a.b_sh = p->b_stride[2];
    a.o_sb = p->output_stride[0];
    a.o_st = p->output_stride[1];
    a.o_sh = p->output_stride[2];
    a.ns_sb = p->new_state_stride[0];
    a.ns_sh = p->new_state_stride[1];
    a.ns_sv = p->new_state_stride[2];
    a.A_log_s = p->A_log_stride;
    a.dt_s = p->dt_bias_stride;
    a.B = B;
    a.T = T;
    a.HV = HV;
    a.ratio = HV / HQK;
    a.scale = p->scale;

    const int64_t nstates = (int64_t)B * T * HV;  // one grid slice per token
    hipStream_t st = (hipStream_t)stream;
    // variant (tuning sweeps): workgroup size x lanes per state row x rows per lane
    // x non-temporal hint; 0 is the default.
    switch (p->variant) {
    case 1: return launch_cfg<256, 8, 2, true>(a, nstates, st);
    case 2: return launch_cfg<256, 8, 4, true>(a, nstates, st);
    case 3: return launch_cfg<256, 8, 1, false>(a, nstates, st);
    case 4: return launch_cfg<256, 16, 1, true>(a, nstates, st);
    case 5: return launch_cfg<128, 8, 1, true>(a, nstates, st);
    case 6: return launch_cfg<128, 16, 1, true>(a, nstates, st);
    case 7: return launch_cfg<256, 16, 2, true>(a, nstates, st);
    case 8: return launch_cfg<64, 8, 1, true>(a, nstates, st);
    default: return launch_cfg<256, 8, 1, true>(a, nstates, st);
    }

}
