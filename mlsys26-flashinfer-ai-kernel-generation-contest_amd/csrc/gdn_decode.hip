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
// DPP reductions. The kernel template also takes other workgroup sizes, 16 lanes per
// row and several rows per lane; only the shape above is instantiated.
#include "gdn_common.h"

#include <algorithm>

namespace gdn {

// Element strides in I: int32_t when the launcher has checked that every element offset
// fits (shorter prologue: 32-bit products, a smaller argument block), else int64_t.
template <typename I>
struct DecodeArgs {
    const bf16_t *q, *k, *v;
    const float *state;
    const float *A_log;
    const bf16_t *a;
    const float *dt_bias;
    const bf16_t *b;
    bf16_t *out;
    float *new_state;
    I q_sb, q_st, q_sh, k_sb, k_st, k_sh, v_sb, v_st, v_sh;
    I st_sb, st_sh, st_sv;
    I a_sb, a_st, a_sh, b_sb, b_st, b_sh;
    I o_sb, o_st, o_sh;
    I ns_sb, ns_sh, ns_sv;
    I A_log_s, dt_s;
    int T;
    int b0;          // first sequence of this launch (grids hold at most 65535 sequences)
    uint32_t gmul;   // h / ratio == umulhi(h, gmul) + h * g_is_h for every h < 65536
    uint32_t g_is_h;
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
    static_assert(LPR == 8 || LPR == 16, "8 or 16 lanes per state row");
    if constexpr (LPR == 8)
        return group8_sum(x);
    else
        return group16_sum(x);
}

// THREADS lanes per workgroup, LPR lanes per state row (8 or 16), RPT rows per lane.
// Lane s of a row owns the float4 column groups 4s + 4*LPR*j, j < NV4.
// Grid (kNVT * T, HV, sequences of this launch): no index needs a division (kNVT is a
// power of two), so the per-wave prologue before the first load stays short.
template <int THREADS, int LPR, int RPT, bool NT, bool HAS_STATE, typename I>
__global__ __launch_bounds__(THREADS) void gdn_decode_kernel(DecodeArgs<I> p)
{
    constexpr int kRowsPerPass = THREADS / LPR;
    constexpr int kNV4 = kD / (4 * LPR);             // float4 per lane per row
    constexpr int kNVT = kD / (kRowsPerPass * RPT);  // workgroups per state
    constexpr int kCols = 4 * kNV4;                  // columns per lane
    static_assert((kNVT & (kNVT - 1)) == 0, "row blocks per state: a power of two");
    const int vt = blockIdx.x % kNVT;
    const int t = blockIdx.x / kNVT;  // token; every token starts from the input state
    const int h = blockIdx.y;
    const I bi = p.b0 + (int)blockIdx.z;
    const I ti = t;
    // GVA: q/k head of this v-head (kernel.py:120) as a multiply-high, no division
    const I g = (I)(__umulhi((uint32_t)h, p.gmul) + (uint32_t)h * p.g_is_h);
    const int tid = threadIdx.x;
    const int s = tid % LPR;
    const int rg = tid / LPR;

    const int v0 = vt * kRowsPerPass * RPT;

    // Load order matters: vector loads return in issue order, so the few small loads
    // (gates, k, q, v) go first and the state stream right after; the gate math then
    // waits only for the small ones while the state is still in flight.
    const uint32_t a_raw = p.a[bi * p.a_sb + ti * p.a_st + (I)h * p.a_sh];
    const uint32_t b_raw = p.b[bi * p.b_sb + ti * p.b_st + (I)h * p.b_sh];
    u32x2 kraw[kNV4], qraw[kNV4];
    {
        const bf16_t *kp = p.k + (bi * p.k_sb + ti * p.k_st + g * p.k_sh + 4 * s);
        const bf16_t *qp = p.q + (bi * p.q_sb + ti * p.q_st + g * p.q_sh + 4 * s);
#pragma unroll
        for (int j = 0; j < kNV4; ++j) {
            kraw[j] = *reinterpret_cast<const u32x2 *>(kp + 4 * LPR * j);
            qraw[j] = *reinterpret_cast<const u32x2 *>(qp + 4 * LPR * j);
        }
    }
    uint32_t vraw[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r)
        vraw[r] = p.v[bi * p.v_sb + ti * p.v_st + (I)h * p.v_sh + (v0 + rg + kRowsPerPass * r)];
    __builtin_amdgcn_sched_barrier(0);

    f32x4 S[RPT][kNV4];
    if constexpr (HAS_STATE) {
        const float *sbase = p.state + (bi * p.st_sb + (I)h * p.st_sh);
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const float *row = sbase + ((I)(v0 + rg + kRowsPerPass * r) * p.st_sv + 4 * s);
#pragma unroll
            for (int j = 0; j < kNV4; ++j)
                S[r][j] = ld4<NT>(row + 4 * LPR * j);
        }
    }
    // the two scheduling barriers pin this issue order
    __builtin_amdgcn_sched_barrier(0);

    // Gates (gdn_decode/solution/triton/kernel.py:123-131), computed while the state
    // is in flight.
    const float A_log = p.A_log[(I)h * p.A_log_s];
    const float dtb = p.dt_bias[(I)h * p.dt_s];
    // base-2 forms on the hardware exp / log / rcp (v_exp_f32, v_log_f32, v_rcp_f32):
    // softplus(x) log2 e = log2(1 + 2^(x log2 e)), alpha = 2^(-e^A_log softplus(x) log2 e)
    constexpr float kLog2e = 1.44269504088896340736f;
    const float x = bf16_to_f32(a_raw) + dtb;
    const float sp2 = x > 20.f ? x * kLog2e
                               : __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(x * kLog2e));
    const float alpha = __builtin_amdgcn_exp2f(-__builtin_amdgcn_exp2f(A_log * kLog2e) * sp2);
    const float beta =
        __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-bf16_to_f32(b_raw) * kLog2e));

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

    float *nbase = p.new_state + (bi * p.ns_sb + (I)h * p.ns_sh);
    bf16_t *obase = p.out + (bi * p.o_sb + ti * p.o_st + (I)h * p.o_sh);
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
        float *nrow = nbase + ((I)row * p.ns_sv + 4 * s);
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

template <typename I>
using DecodeArgs = gdn::DecodeArgs<I>;

template <int THREADS, int LPR, int RPT, bool NT, typename I>
int launch_grid(DecodeArgs<I> a, int B, int HV, hipStream_t stream)
{
    constexpr int kNVT = gdn::kD / ((THREADS / LPR) * RPT);
    const int64_t gx = (int64_t)a.T * kNVT;
    if (gx > 0x7fffffff)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: seq_len %d too large", a.T);
    gdn_begin_launches();
    for (int b0 = 0; b0 < B; b0 += 65535) {
        a.b0 = b0;
        const dim3 grid((unsigned)gx, (unsigned)HV, (unsigned)std::min(65535, B - b0));
        if (a.state)
            hipLaunchKernelGGL((gdn::gdn_decode_kernel<THREADS, LPR, RPT, NT, true, I>), grid,
                               dim3(THREADS), 0, stream, a);
        else
            hipLaunchKernelGGL((gdn::gdn_decode_kernel<THREADS, LPR, RPT, NT, false, I>), grid,
                               dim3(THREADS), 0, stream, a);
        const int rc = gdn_check_launch("gdn_decode_kernel");
        if (rc)
            return rc;
    }
    return GDN_OK;
}

// The int32 form when every stride is in [0, 2^31) and every element offset (the largest
// index of each tensor) stays below 2^31; the int64 form otherwise.
bool fits32(const DecodeArgs<int64_t> &a, int B, int HQK, int HV)
{
    const int64_t lim = int64_t(1) << 31;
    const int64_t st[] = {a.q_sb, a.q_st, a.q_sh, a.k_sb, a.k_st, a.k_sh, a.v_sb, a.v_st,
                          a.v_sh, a.st_sb, a.st_sh, a.st_sv, a.a_sb, a.a_st, a.a_sh, a.b_sb,
                          a.b_st, a.b_sh, a.o_sb, a.o_st, a.o_sh, a.ns_sb, a.ns_sh, a.ns_sv,
                          a.A_log_s, a.dt_s};
    for (int64_t x : st)
        if (x < 0 || x >= lim)
            return false;
    const int64_t b = B - 1, t = a.T - 1, D = gdn::kD - 1;
    auto last = [&](int64_t sb, int64_t stt, int64_t sh, int64_t heads, int64_t inner) {
        return b * sb + t * stt + (heads - 1) * sh + inner;
    };
    return last(a.q_sb, a.q_st, a.q_sh, HQK, D) < lim && last(a.k_sb, a.k_st, a.k_sh, HQK, D) < lim &&
           last(a.v_sb, a.v_st, a.v_sh, HV, D) < lim && last(a.a_sb, a.a_st, a.a_sh, HV, 0) < lim &&
           last(a.b_sb, a.b_st, a.b_sh, HV, 0) < lim && last(a.o_sb, a.o_st, a.o_sh, HV, D) < lim &&
           (!a.state || last(a.st_sb, 0, a.st_sh, HV, D * a.st_sv + D) < lim) &&
           last(a.ns_sb, 0, a.ns_sh, HV, D * a.ns_sv + D) < lim &&
           (int64_t)(HV - 1) * a.A_log_s < lim && (int64_t)(HV - 1) * a.dt_s < lim;
}

template <int THREADS, int LPR, int RPT, bool NT>
int launch_cfg(const DecodeArgs<int64_t> &a, int B, int HQK, int HV, hipStream_t stream)
{
    if (!fits32(a, B, HQK, HV))
        return launch_grid<THREADS, LPR, RPT, NT>(a, B, HV, stream);
    DecodeArgs<int32_t> n;
    n.q = a.q; n.k = a.k; n.v = a.v; n.state = a.state; n.A_log = a.A_log; n.a = a.a;
    n.dt_bias = a.dt_bias; n.b = a.b; n.out = a.out; n.new_state = a.new_state;
    n.q_sb = (int32_t)a.q_sb; n.q_st = (int32_t)a.q_st; n.q_sh = (int32_t)a.q_sh;
    n.k_sb = (int32_t)a.k_sb; n.k_st = (int32_t)a.k_st; n.k_sh = (int32_t)a.k_sh;
    n.v_sb = (int32_t)a.v_sb; n.v_st = (int32_t)a.v_st; n.v_sh = (int32_t)a.v_sh;
    n.st_sb = (int32_t)a.st_sb; n.st_sh = (int32_t)a.st_sh; n.st_sv = (int32_t)a.st_sv;
    n.a_sb = (int32_t)a.a_sb; n.a_st = (int32_t)a.a_st; n.a_sh = (int32_t)a.a_sh;
    n.b_sb = (int32_t)a.b_sb; n.b_st = (int32_t)a.b_st; n.b_sh = (int32_t)a.b_sh;
    n.o_sb = (int32_t)a.o_sb; n.o_st = (int32_t)a.o_st; n.o_sh = (int32_t)a.o_sh;
    n.ns_sb = (int32_t)a.ns_sb; n.ns_sh = (int32_t)a.ns_sh; n.ns_sv = (int32_t)a.ns_sv;
    n.A_log_s = (int32_t)a.A_log_s; n.dt_s = (int32_t)a.dt_s;
    n.T = a.T; n.b0 = 0; n.gmul = a.gmul; n.g_is_h = a.g_is_h; n.scale = a.scale;
    return launch_grid<THREADS, LPR, RPT, NT>(n, B, HV, stream);
}

bool aligned(const void *p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

}  // namespace

extern "C" int gdn_decode_launch(const gdn_decode_params *p, void *stream)
{
    gdn_begin_call();
    if (!p || p->struct_size != (int32_t)sizeof(gdn_decode_params))
        return gdn_set_error(GDN_EINVAL, "gdn_decode: params NULL or struct_size mismatch");
    const int B = p->batch, T = p->seq_len, HQK = p->num_qk_heads, HV = p->num_v_heads,
              D = p->head_size;
    if (B < 0 || HQK <= 0 || HV <= 0 || HV % HQK != 0)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: bad sizes B=%d HQK=%d HV=%d", B, HQK, HV);
    if (HV > 65535)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: num_v_heads %d above 65535", HV);
    if (D != 128)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: head_size %d unsupported (128 only)", D);
    if (T < 1)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: seq_len %d must be >= 1", T);
    if (p->variant != 0)
        return gdn_set_error(GDN_EINVAL, "gdn_decode: variant %d unknown (0 only)", p->variant);
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

    DecodeArgs<int64_t> a;
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
    a.T = T;
    a.scale = p->scale;
    a.b0 = 0;
    // h / ratio for h < HV <= 65535: ratio 1 is h itself; otherwise m = ceil(2^32 / ratio)
    // = (2^32 + e) / ratio with 0 <= e < ratio, and umulhi(h, m) = floor(h / ratio +
    // h e / (2^32 ratio)) = h / ratio since h e < h ratio < 2^32
    const uint32_t ratio = (uint32_t)(HV / HQK);
    a.g_is_h = ratio == 1;
    a.gmul = ratio == 1 ? 0u : (uint32_t)(((uint64_t(1) << 32) + ratio - 1) / ratio);

    // 256 lanes, 8 lanes per state row, one row per lane, non-temporal state loads and
    // stores: the fastest of the swept shapes at B = 1, 64 and 256 on MI355X
    return launch_cfg<256, 8, 1, true>(a, B, HQK, HV, (hipStream_t)stream);
}
