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
// Thread mapping: a workgroup of 256 lanes covers 32 state rows per pass; each
// row is spread over 8 consecutive lanes and each lane owns 16 columns as four
// float4 at columns 4s + 32j (s = lane % 8, j = 0..3), so one load instruction
// of a wavefront covers eight full 128-byte row segments. Row sums are 8-lane
// DPP reductions. RPT passes per workgroup -> 32*RPT rows per workgroup.
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
    int64_t q_sb, q_sh, k_sb, k_sh, v_sb, v_sh;
    int64_t st_sb, st_sh, st_sv;
    int64_t a_sb, a_sh, b_sb, b_sh;
    int64_t o_sb, o_sh;
    int64_t ns_sb, ns_sh, ns_sv;
    int64_t A_log_s, dt_s;
    int HV, ratio;
    float scale;
};

constexpr int kDecThreads = 256;
constexpr int kDecRowsPerPass = kDecThreads / 8;
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

// Loads 4 consecutive bf16 (8 bytes) and widens them.
__device__ __forceinline__ void ld_bf16x4(const bf16_t *p, float *dst)
{
    u32x2 w = *reinterpret_cast<const u32x2 *>(p);
    dst[0] = bf16lo(w.x);
    dst[1] = bf16hi(w.x);
    dst[2] = bf16lo(w.y);
    dst[3] = bf16hi(w.y);
}

template <int RPT, bool NT, bool HAS_STATE>
__global__ __launch_bounds__(kDecThreads) void gdn_decode_kernel(DecodeArgs p)
{
    constexpr int kNVT = kD / (kDecRowsPerPass * RPT);  // workgroups per state
    const int bid = blockIdx.x;
    const int vt = bid % kNVT;
    const int bh = bid / kNVT;
    const int h = bh % p.HV;
    const int bi = bh / p.HV;
    const int g = h / p.ratio;  // GVA: q/k head of this v-head (kernel.py:120)
    const int tid = threadIdx.x;
    const int s = tid & 7;
    const int rg = tid >> 3;

    // Gates (gdn_decode/solution/triton/kernel.py:123-131).
    const float A_log = p.A_log[h * p.A_log_s];
    const float dtb = p.dt_bias[h * p.dt_s];
    const float av = bf16_to_f32(p.a[bi * p.a_sb + h * p.a_sh]);
    const float bv = bf16_to_f32(p.b[bi * p.b_sb + h * p.b_sh]);
    const float x = av + dtb;
    const float sp = x > 20.f ? x : logf(1.f + expf(x));
    const float alpha = expf(-expf(A_log) * sp);
    const float beta = 1.f / (1.f + expf(-bv));

    const int v0 = vt * kDecRowsPerPass * RPT;

    // Issue the state loads first: they are the bytes that matter.
    f32x4 S[RPT][4];
    if constexpr (HAS_STATE) {
        const float *sbase = p.state + bi * p.st_sb + h * p.st_sh;
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const float *row = sbase + (int64_t)(v0 + rg + kDecRowsPerPass * r) * p.st_sv + 4 * s;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                S[r][j] = ld4<NT>(row + 32 * j);
        }
    }

    float kk[16], qq[16];
    {
        const bf16_t *kp = p.k + bi * p.k_sb + g * p.k_sh + 4 * s;
        const bf16_t *qp = p.q + bi * p.q_sb + g * p.q_sh + 4 * s;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ld_bf16x4(kp + 32 * j, kk + 4 * j);
            ld_bf16x4(qp + 32 * j, qq + 4 * j);
        }
    }
    float vrow[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r)
        vrow[r] = bf16_to_f32(p.v[bi * p.v_sb + h * p.v_sh + v0 + rg + kDecRowsPerPass * r]);

    float kq = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        kq = fmaf(kk[i], qq[i], kq);
    kq = group8_sum(kq);

    float *nbase = p.new_state + bi * p.ns_sb + h * p.ns_sh;
    bf16_t *obase = p.out + bi * p.o_sb + h * p.o_sh;
    const float omb = 1.f - beta;
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int row = v0 + rg + kDecRowsPerPass * r;
        float sk = 0.f, sq = 0.f;
        if constexpr (HAS_STATE) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sk = fmaf(S[r][j][e], kk[4 * j + e], sk);
                    sq = fmaf(S[r][j][e], qq[4 * j + e], sq);
                }
            }
            sk = group8_sum(sk);
            sq = group8_sum(sq);
        }
        const float u = alpha * sk;                  // (alpha S) k      kernel.py:165-166
        const float nv = beta * vrow[r] + omb * u;   // kernel.py:167
        const float d = nv - u;                      // kernel.py:168
        const float o = fmaf(alpha, sq, d * kq);     // (alpha S + d k^T) q
        float *nrow = nbase + (int64_t)row * p.ns_sv + 4 * s;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sv = HAS_STATE ? S[r][j][e] : 0.f;
                w[e] = fmaf(alpha, sv, d * kk[4 * j + e]);  // kernel.py:169
            }
            st4<NT>(nrow + 32 * j, w);
        }
        if (s == 0)
            obase[row] = (bf16_t)f32_to_bf16(p.scale * o);  // kernel.py:216-218
    }
}

}  // namespace gdn

namespace {

using gdn::DecodeArgs;

template <int RPT, bool NT>
int launch_rpt(const DecodeArgs &a, int64_t nstates, hipStream_t stream)
{
    constexpr int kNVT = gdn::kD / (gdn::kDecRowsPerPass * RPT);
    const int64_t blocks = (int64_t)nstates * kNVT;
    if (blocks > 0x7fffffff)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: grid too large (%lld workgroups)",
                             (long long)blocks);
    if (a.state)
        hipLaunchKernelGGL((gdn::gdn_decode_kernel<RPT, NT, true>), dim3((unsigned)blocks),
                           dim3(gdn::kDecThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((gdn::gdn_decode_kernel<RPT, NT, false>), dim3((unsigned)blocks),
                           dim3(gdn::kDecThreads), 0, stream, a);
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
    if (T != 1)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: seq_len %d unsupported (1 only)", T);
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
    a.q_sh = p->q_stride[2];
    a.k_sb = p->k_stride[0];
    a.k_sh = p->k_stride[2];
    a.v_sb = p->v_stride[0];
    a.v_sh = p->v_stride[2];
    a.st_sb = p->state_stride[0];
    a.st_sh = p->state_stride[1];
    a.st_sv = p->state_stride[2];
    a.a_sb = p->a_stride[0];
    a.a_sh = p->a_stride[2];
    a.b_sb = p->b_stride[0];
    a.b_sh = p->b_stride[2];
    a.o_sb = p->output_stride[0];
    a.o_sh = p->output_stride[2];
    a.ns_sb = p->new_state_stride[0];
    a.ns_sh = p->new_state_stride[1];
    a.ns_sv = p->new_state_stride[2];
    a.A_log_s = p->A_log_stride;
    a.dt_s = p->dt_bias_stride;
    a.HV = HV;
    a.ratio = HV / HQK;
    a.scale = p->scale;

    const int64_t nstates = (int64_t)B * HV;
    hipStream_t st = (hipStream_t)stream;
    // variant: rows per thread x non-temporal hint. 0 (the default) = 1 row per thread,
    // non-temporal: the fastest on MI355X at B = 1, 64 and 256.
    switch (p->variant) {
    case 1: return launch_rpt<2, true>(a, nstates, st);
    case 2: return launch_rpt<4, true>(a, nstates, st);
    case 3: return launch_rpt<1, false>(a, nstates, st);
    case 4: return launch_rpt<2, false>(a, nstates, st);
    case 5: return launch_rpt<4, false>(a, nstates, st);
    default: return launch_rpt<1, true>(a, nstates, st);
    }

}
