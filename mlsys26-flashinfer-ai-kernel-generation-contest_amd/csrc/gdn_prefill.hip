// Packed variable-length Gated DeltaNet prefill for gfx950: chunked WY/UT form,
// C = 64 tokens per chunk, bf16 MFMA with fp32 accumulation.
//
// Per chunk of one sequence and v-head h (q/k head g = h / ratio), with start
// state S0 (k-last, S[v,k]) and L_t = sum_{i<=t} log alpha_i inside the chunk:
//   A[t,j] = beta_t exp(L_t - L_j) (k_t . k_j)  (j < t),    T = (I + A)^-1
//   U      = T (beta * (V - exp(L) * (K S0^T)))               (pseudo-values)
//   O      = scale * (exp(L) * (Q S0^T) + P U),  P[t,j] = exp(L_t - L_j) (q_t . k_j), j <= t
//   S_end  = exp(L_C) S0 + (exp(L_C - L) * U)^T K
// (gdn_prefill/solution/triton/kernel.py:60-79; Yang et al. 2024, "Parallelizing
// Linear Transformers with the Delta Rule over Sequence Length" / "Gated Delta
// Networks"). Only non-positive log differences are exponentiated, so strong
// decay underflows to 0 instead of overflowing; no clamping.
//
// Three launches on the caller's stream:
//   plan  (1 + Z workgroups): sequence -> chunk tables from cu_seqlens on the
//         device (no host sync), longest-first sequence order, and zero-fill of
//         output rows that belong to no sequence.
//   prep  (chunks x q/k heads): K K^T and Q K^T on MFMA, gates, cumulative log
//         decay, T = (I + A)^-1 (fp32: 16x16 diagonal blocks by substitution,
//         off-diagonal blocks on fp32 MFMA), P; writes per (chunk, v-head) records.
//   scan  (sequences x v-heads x 8 V-tiles): one workgroup owns 16 state rows of
//         one (sequence, v-head) and walks its chunks in order, state in
//         registers. fp32-valued operands on the state path (S0, R, T, U) are split
//         into bf16 hi + lo halves so the state keeps ~2^-16 relative accuracy.
#include "gdn_common.h"

namespace gdn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// hi = bf16(x), lo = bf16(x - hi)
__device__ __forceinline__ void split_bf16(float x, uint32_t &hi, uint32_t &lo)
{
    hi = f32_to_bf16(x);
    lo = f32_to_bf16(x - bf16_to_f32(hi));
}

constexpr int kC = 64;   // chunk length
constexpr int kDK = 128; // head size
constexpr int kLdK = 136; // padded LDS row (bf16) for 64 x 128 tiles
constexpr int kLdT = 72;  // padded LDS row (bf16) for 16 x 64 tiles

// Per (chunk, v-head) record in the workspace.
constexpr int kRecThi = 0;       // bf16 [64][64]  T = (I + A)^-1, high half
constexpr int kRecTlo = 8192;    // bf16 [64][64]  low half
constexpr int kRecP = 16384;     // bf16 [64][64]  P (decayed, causal Q K^T)
constexpr int kRecGates = 24576; // f32 beta[64], gamma[64], dec[64], gammaC
constexpr int kRecBytes = 25600;

__device__ __forceinline__ int64_t load_cu(const void *cu, int cu64, int i)
{
    return cu64 ? ((const int64_t *)cu)[i] : (int64_t)((const int32_t *)cu)[i];
}

// ------------------------------------------------------------------------- plan
struct PlanArgs {
    const void *cu;
    int cu64, N, T, HO, nc;  // nc: chunk-table capacity (workspace bound)
    int32_t *header, *chunk_tok0, *chunk_len, *seq_chunk0, *seq_order, *seq_tok0, *seq_len;
    bf16_t *out;
    int64_t o_st, o_sh;
};

constexpr int kPlanSortMax = 512;

__global__ __launch_bounds__(256) void gdn_prefill_plan_kernel(PlanArgs p)
{
    const int tid = threadIdx.x;
    if (blockIdx.x == 0) {
        // Chunk counts are clamped so that malformed (non-monotone) cu_seqlens can
        // never index past the chunk tables or records sized for nc chunks; for
        // valid input sum(ceil(len / C)) <= ceil(T / C) + N = nc always holds.
        __shared__ int64_t scan[256];
        __shared__ int32_t s_nck[kPlanSortMax];
        __shared__ int64_t s_carry;
        if (tid == 0)
            s_carry = 0;
        __syncthreads();
        for (int base = 0; base < p.N; base += 256) {
            const int n = base + tid;
            int nck = 0, t0 = 0, ln = 0;
            if (n < p.N) {
                int64_t a = load_cu(p.cu, p.cu64, n), b = load_cu(p.cu, p.cu64, n + 1);
                a = a < 0 ? 0 : (a > p.T ? p.T : a);  // clamp: never index outside [0, T)
                b = b < a ? a : (b > p.T ? p.T : b);
                t0 = (int)a;
                ln = (int)(b - a);
                nck = (ln + kC - 1) / kC;
                p.seq_tok0[n] = t0;
                p.seq_len[n] = ln;
                if (n < kPlanSortMax)
                    s_nck[n] = nck;
            }
            scan[tid] = nck;
            __syncthreads();
            for (int off = 1; off < 256; off <<= 1) {
                const int64_t add = tid >= off ? scan[tid - off] : 0;
                __syncthreads();
                scan[tid] += add;
                __syncthreads();
            }
            const int64_t first = s_carry + scan[tid] - nck;
            if (n < p.N) {
                p.seq_chunk0[n] = (int32_t)(first < p.nc ? first : p.nc);
                for (int i = 0; i < nck && first + i < p.nc; ++i) {
                    p.chunk_tok0[first + i] = t0 + i * kC;
                    p.chunk_len[first + i] = min(kC, ln - i * kC);
                }
            }
            __syncthreads();
            if (tid == 255)
                s_carry += scan[255];
            __syncthreads();
        }
        if (tid == 0) {
            const int32_t total = (int32_t)(s_carry < p.nc ? s_carry : p.nc);
            p.seq_chunk0[p.N] = total;
            p.header[0] = total;
        }
        // Longest-first order (identity when N is large).
        if (p.N <= kPlanSortMax) {
            for (int n = tid; n < p.N; n += 256) {
                const int mine = s_nck[n];
                int rank = 0;
                for (int m = 0; m < p.N; ++m) {
                    const int o = s_nck[m];
                    rank += (o > mine) || (o == mine && m < n);
                }
                p.seq_order[rank] = n;
            }
        } else {
            for (int n = tid; n < p.N; n += 256)
                p.seq_order[n] = n;
        }
        return;
    }
    // Zero-fill output rows of tokens outside [cu[0], cu[N]).
    int64_t g0 = p.N > 0 ? load_cu(p.cu, p.cu64, 0) : p.T;
    g0 = g0 < 0 ? 0 : (g0 > p.T ? p.T : g0);
    int64_t g1 = p.N > 0 ? load_cu(p.cu, p.cu64, p.N) : p.T;
    g1 = g1 < g0 ? g0 : (g1 > p.T ? p.T : g1);
    const int64_t gap = g0 + (p.T - g1);
    const int64_t vec_per_tok = (int64_t)p.HO * (kDK / 8);
    const int64_t total = gap * vec_per_tok;
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int64_t i = (int64_t)(blockIdx.x - 1) * 256 + tid; i < total;
         i += (int64_t)(gridDim.x - 1) * 256) {
        const int64_t gt = i / vec_per_tok;
        const int64_t rem = i % vec_per_tok;
        const int64_t tok = gt < g0 ? gt : g1 + (gt - g0);
        const int64_t hh = rem / (kDK / 8);
        const int64_t col = (rem % (kDK / 8)) * 8;
        *(u32x4 *)(p.out + tok * p.o_st + hh * p.o_sh + col) = z;
    }
}

// ------------------------------------------------------------------------- prep
struct PrepArgs {
    const bf16_t *q, *k, *a, *b;
    const float *A_log, *dt_bias;
    int64_t q_st, q_sh, k_st, k_sh, a_st, a_sh, b_st, b_sh, A_log_s, dt_s;
    const int32_t *header, *chunk_tok0, *chunk_len;
    char *records;
    int HV, ratio;
};

__global__ __launch_bounds__(256) void gdn_prefill_prep_kernel(PrepArgs p)
{
    const int c = blockIdx.x;
    const int g = blockIdx.y;
    if (c >= p.header[0])
        return;
    const int tok0 = p.chunk_tok0[c];
    const int len = p.chunk_len[c];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lr = l & 15, lg = l >> 4;

    __shared__ __align__(16) bf16_t Ks[kC][kLdK];
    __shared__ __align__(16) bf16_t Qs[kC][kLdK];
    __shared__ __align__(16) float As[kC][kC + 4];
    __shared__ __align__(16) float Ts[kC][kC + 4];
    __shared__ __align__(16) float Ms[4][16][17];
    __shared__ float Lg[kC], Bt[kC];

    // K, Q chunk rows -> LDS (zero rows past the chunk's length).
    for (int s = tid; s < kC * (kDK / 8); s += 256) {
        const int row = s >> 4, col = (s & 15) * 8;
        u32x4 kv = {0u, 0u, 0u, 0u}, qv = {0u, 0u, 0u, 0u};
        if (row < len) {
            kv = *(const u32x4 *)(p.k + (int64_t)(tok0 + row) * p.k_st + g * p.k_sh + col);
            qv = *(const u32x4 *)(p.q + (int64_t)(tok0 + row) * p.q_st + g * p.q_sh + col);
        }
        *(u32x4 *)&Ks[row][col] = kv;
        *(u32x4 *)&Qs[row][col] = qv;
    }
    __syncthreads();

    // Row block w of K K^T and Q K^T (only tiles on or below the diagonal).
    f32x4 kk[4], qk[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
        kk[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
        qk[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (jt <= w) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const u32x4 ak = *(const u32x4 *)&Ks[16 * w + lr][ks * 32 + 8 * lg];
                const u32x4 aq = *(const u32x4 *)&Qs[16 * w + lr][ks * 32 + 8 * lg];
                const u32x4 bk = *(const u32x4 *)&Ks[16 * jt + lr][ks * 32 + 8 * lg];
                kk[jt] = mfma_bf16(ak, bk, kk[jt]);
                qk[jt] = mfma_bf16(aq, bk, qk[jt]);
            }
        }
    }

    for (int hh = 0; hh < p.ratio; ++hh) {
        const int h = g * p.ratio + hh;
        char *rec = p.records + ((int64_t)c * p.HV + h) * kRecBytes;
        float *gates = (float *)(rec + kRecGates);

        // Gates and the in-chunk cumulative log decay (wave 0, one lane per token).
        if (w == 0) {
            float la = 0.f, bt = 0.f;
            if (l < len) {
                const float A_log = p.A_log[h * p.A_log_s];
                const float dtb = p.dt_bias[h * p.dt_s];
                const float x = bf16_to_f32(p.a[(int64_t)(tok0 + l) * p.a_st + h * p.a_sh]) + dtb;
                const float sp = x > 20.f ? x : logf(1.f + expf(x));
                la = -expf(A_log) * sp;
                const float bv = bf16_to_f32(p.b[(int64_t)(tok0 + l) * p.b_st + h * p.b_sh]);
                bt = 1.f / (1.f + expf(-bv));
            }
            float L = la;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const float y = __shfl_up(L, off, 64);
                if (l >= off)
                    L += y;
            }
            const float Lend = __shfl(L, 63, 64);
            Lg[l] = L;
            Bt[l] = bt;
            gates[l] = bt;
            gates[64 + l] = expf(L);
            gates[128 + l] = expf(Lend - L);
            if (l == 0)
                gates[192] = expf(Lend);
        }
        __syncthreads();

        // A (strictly lower, fp32) -> LDS; P (lower incl., bf16) -> record.
        bf16_t *Prec = (bf16_t *)(rec + kRecP);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 16 * w + 4 * lg + i;
                const int j = 16 * jt + lr;
                float av = 0.f, pv = 0.f;
                if (jt <= w && j <= t) {
                    const float e = expf(Lg[t] - Lg[j]);
                    pv = e * qk[jt][i];
                    if (j < t)
                        av = Bt[t] * e * kk[jt][i];
                }
                As[t][j] = av;
                Prec[t * kC + j] = (bf16_t)f32_to_bf16(pv);
            }
        }
        __syncthreads();

        // Diagonal 16x16 blocks of T by forward substitution: wave 0, lane =
        // (block, column).
        if (w == 0) {
            const int blk = l >> 4, col = l & 15, o = 16 * blk;
            float x[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float acc = (r == col) ? 1.f : 0.f;
#pragma unroll
                for (int j = 0; j < r; ++j)
                    acc = fmaf(-As[o + r][o + j], x[j], acc);
                x[r] = acc;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r)
                Ts[o + r][o + col] = x[r];
        } else {
            // zero the strictly-upper blocks (T is lower triangular)
            for (int e = tid - 64; e < kC * kC; e += 192) {
                const int r = e >> 6, cc = e & 63;
                if ((cc >> 4) > (r >> 4))
                    Ts[r][cc] = 0.f;
            }
        }
        __syncthreads();

        // Off-diagonal blocks, one block diagonal at a time:
        //   T_ij = -T_ii * sum_{m=j}^{i-1} A_im T_mj      (fp32 MFMA 16x16x4)
        for (int d = 1; d < 4; ++d) {
            const int i = w + d, j = w;
            const bool active = i < 4;
            if (active) {
                f32x4 M = {0.f, 0.f, 0.f, 0.f};
                for (int m = j; m < i; ++m) {
#pragma unroll
                    for (int k4 = 0; k4 < 4; ++k4) {
                        const float av = As[16 * i + lr][16 * m + 4 * k4 + lg];
                        const float bv = Ts[16 * m + 4 * k4 + lg][16 * j + lr];
                        M = mfma_f32(av, bv, M);
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    Ms[w][4 * lg + e][lr] = M[e];
            }
            __syncthreads();
            if (active) {
                f32x4 R = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k4 = 0; k4 < 4; ++k4) {
                    const float av = Ts[16 * i + lr][16 * i + 4 * k4 + lg];
                    const float bv = Ms[w][4 * k4 + lg][lr];
                    R = mfma_f32(av, bv, R);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    Ts[16 * i + 4 * lg + e][16 * j + lr] = -R[e];
            }
            __syncthreads();
        }

        // T -> record as bf16 hi / lo halves, row-major [64][64].
        {
            const int row = tid >> 2, c0 = (tid & 3) * 16;
            bf16_t *thi = (bf16_t *)(rec + kRecThi) + row * kC + c0;
            bf16_t *tlo = (bf16_t *)(rec + kRecTlo) + row * kC + c0;
            uint32_t hw[8], lw[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                uint32_t h0, l0, h1, l1;
                split_bf16(Ts[row][c0 + 2 * e], h0, l0);
                split_bf16(Ts[row][c0 + 2 * e + 1], h1, l1);
                hw[e] = h0 | (h1 << 16);
                lw[e] = l0 | (l1 << 16);
            }
            *(u32x4 *)thi = u32x4{hw[0], hw[1], hw[2], hw[3]};
            *(u32x4 *)(thi + 8) = u32x4{hw[4], hw[5], hw[6], hw[7]};
            *(u32x4 *)tlo = u32x4{lw[0], lw[1], lw[2], lw[3]};
            *(u32x4 *)(tlo + 8) = u32x4{lw[4], lw[5], lw[6], lw[7]};
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------- scan
struct ScanArgs {
    const bf16_t *q, *k, *v;
    const float *state;
    float *new_state;
    bf16_t *out;
    int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh;
    int64_t st_sn, st_sh, st_sv, ns_sn, ns_sh, ns_sv;
    const int32_t *header, *seq_chunk0, *seq_order, *seq_tok0, *seq_len;
    const char *records;
    int HQK, HV, ratio, ngroups;
    float scale;
};

__global__ __launch_bounds__(256) void gdn_prefill_scan_kernel(ScanArgs p)
{
    // Workgroups of one (sequence, q/k head) group share K, Q, T and P through L2:
    // place them on one XCD (workgroup ids are dealt to the 8 XCDs round-robin).
    const int pid = blockIdx.x, xcd = pid & 7, slot = pid >> 3;
    const int gsz = 8 * p.ratio;
    const int wi = slot % gsz;
    const int grp = (slot / gsz) * 8 + xcd;
    if (grp >= p.ngroups)
        return;
    const int n = p.seq_order[grp / p.HQK];
    const int g = grp % p.HQK;
    const int h = g * p.ratio + wi / 8;
    const int v0 = (wi % 8) * 16;
    const int tok0 = p.seq_tok0[n], len = p.seq_len[n], c0 = p.seq_chunk0[n];
    // records exist only for chunk ids < header[0] (see the plan kernel's clamp)
    const int nck = min((len + kC - 1) / kC, max(p.header[0] - c0, 0));

    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lr = l & 15, lg = l >> 4;

    __shared__ __align__(16) bf16_t Ks[kC][kLdK];
    __shared__ __align__(16) bf16_t Shi[16][kLdK];
    __shared__ __align__(16) bf16_t Slo[16][kLdK];
    __shared__ __align__(16) bf16_t RThi[16][kLdT];
    __shared__ __align__(16) bf16_t RTlo[16][kLdT];
    __shared__ __align__(16) bf16_t UThi[16][kLdT];
    __shared__ __align__(16) bf16_t WThi[16][kLdT];
    __shared__ __align__(16) bf16_t WTlo[16][kLdT];

    // State tile rows v0..v0+15 in MFMA C layout: Sreg[j][i] = S[v0 + 4 lg + i][16 (2w + j) + lr].
    f32x4 Sreg[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int vv = v0 + 4 * lg + i, kc = 16 * (2 * w + j) + lr;
            Sreg[j][i] = p.state ? p.state[n * p.st_sn + h * p.st_sh + vv * p.st_sv + kc] : 0.f;
        }
    auto stage_state = [&]() {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t hi, lo;
                split_bf16(Sreg[j][i], hi, lo);
                Shi[4 * lg + i][16 * (2 * w + j) + lr] = (bf16_t)hi;
                Slo[4 * lg + i][16 * (2 * w + j) + lr] = (bf16_t)lo;
            }
    };
    stage_state();

    for (int c = 0; c < nck; ++c) {
        const int tokc = tok0 + c * kC;
        const int lenc = min(kC, len - c * kC);
        const char *rec = p.records + ((int64_t)(c0 + c) * p.HV + h) * kRecBytes;
        const float *gates = (const float *)(rec + kRecGates);

        // (0) K chunk -> LDS
        for (int s = tid; s < kC * (kDK / 8); s += 256) {
            const int row = s >> 4, col = (s & 15) * 8;
            u32x4 kv = {0u, 0u, 0u, 0u};
            if (row < lenc)
                kv = *(const u32x4 *)(p.k + (int64_t)(tokc + row) * p.k_st + g * p.k_sh + col);
            *(u32x4 *)&Ks[row][col] = kv;
        }
        __syncthreads();

        // (a) X = K S0^T for tokens 16w..16w+15 (S0 as hi + lo)
        f32x4 X = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const u32x4 a = *(const u32x4 *)&Ks[16 * w + lr][ks * 32 + 8 * lg];
            const u32x4 bh = *(const u32x4 *)&Shi[lr][ks * 32 + 8 * lg];
            const u32x4 bl = *(const u32x4 *)&Slo[lr][ks * 32 + 8 * lg];
            X = mfma_bf16(a, bh, X);
            X = mfma_bf16(a, bl, X);
        }
        // (b) R = beta (V - gamma X)  -> LDS as R^T (hi, lo)
        float gam[4];
        {
            uint32_t rh[4], rl[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 16 * w + 4 * lg + i;
                const float vv = t < lenc
                    ? bf16_to_f32(p.v[(int64_t)(tokc + t) * p.v_st + h * p.v_sh + v0 + lr])
                    : 0.f;
                gam[i] = gates[64 + t];
                const float r = gates[t] * (vv - gam[i] * X[i]);
                split_bf16(r, rh[i], rl[i]);
            }
            *(u32x2 *)&RThi[lr][16 * w + 4 * lg] = u32x2{rh[0] | (rh[1] << 16), rh[2] | (rh[3] << 16)};
            *(u32x2 *)&RTlo[lr][16 * w + 4 * lg] = u32x2{rl[0] | (rl[1] << 16), rl[2] | (rl[3] << 16)};
        }
        __syncthreads();

        // (c) U = T R  (T, R as hi + lo; three products)
        f32x4 U = {0.f, 0.f, 0.f, 0.f};
        {
            const bf16_t *thi = (const bf16_t *)(rec + kRecThi);
            const bf16_t *tlo = (const bf16_t *)(rec + kRecTlo);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                if (ks == 1 && w < 2)
                    continue;  // T rows < 32 have no entries in columns >= 32
                const u32x4 ah = *(const u32x4 *)(thi + (16 * w + lr) * kC + ks * 32 + 8 * lg);
                const u32x4 al = *(const u32x4 *)(tlo + (16 * w + lr) * kC + ks * 32 + 8 * lg);
                const u32x4 bh = *(const u32x4 *)&RThi[lr][ks * 32 + 8 * lg];
                const u32x4 bl = *(const u32x4 *)&RTlo[lr][ks * 32 + 8 * lg];
                U = mfma_bf16(ah, bh, U);
                U = mfma_bf16(ah, bl, U);
                U = mfma_bf16(al, bh, U);
            }
            uint32_t uh[4], wh[4], wl[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 16 * w + 4 * lg + i;
                uh[i] = f32_to_bf16(U[i]);
                split_bf16(gates[128 + t] * U[i], wh[i], wl[i]);
            }
            *(u32x2 *)&UThi[lr][16 * w + 4 * lg] = u32x2{uh[0] | (uh[1] << 16), uh[2] | (uh[3] << 16)};
            *(u32x2 *)&WThi[lr][16 * w + 4 * lg] = u32x2{wh[0] | (wh[1] << 16), wh[2] | (wh[3] << 16)};
            *(u32x2 *)&WTlo[lr][16 * w + 4 * lg] = u32x2{wl[0] | (wl[1] << 16), wl[2] | (wl[3] << 16)};
        }
        __syncthreads();

        // (d) O = scale (gamma Q S0^T + P U) for tokens 16w..16w+15
        {
            f32x4 Oi = {0.f, 0.f, 0.f, 0.f}, Oa = {0.f, 0.f, 0.f, 0.f};
            const int trow = 16 * w + lr;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                u32x4 aq = {0u, 0u, 0u, 0u};
                if (trow < lenc)
                    aq = *(const u32x4 *)(p.q + (int64_t)(tokc + trow) * p.q_st + g * p.q_sh +
                                          ks * 32 + 8 * lg);
                const u32x4 bh = *(const u32x4 *)&Shi[lr][ks * 32 + 8 * lg];
                Oi = mfma_bf16(aq, bh, Oi);
            }
            const bf16_t *prec = (const bf16_t *)(rec + kRecP);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                if (ks == 1 && w < 2)
                    continue;
                const u32x4 ap = *(const u32x4 *)(prec + trow * kC + ks * 32 + 8 * lg);
                const u32x4 bu = *(const u32x4 *)&UThi[lr][ks * 32 + 8 * lg];
                Oa = mfma_bf16(ap, bu, Oa);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 16 * w + 4 * lg + i;
                if (t < lenc)
                    p.out[(int64_t)(tokc + t) * p.o_st + h * p.o_sh + v0 + lr] =
                        (bf16_t)f32_to_bf16(p.scale * fmaf(gam[i], Oi[i], Oa[i]));
            }
        }

        // (e) S = gammaC S + W^T K over this wave's 32 state columns
        {
            const float gC = gates[192];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int kc = 16 * (2 * w + j) + lr;
                f32x4 dS = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const u32x4 awh = *(const u32x4 *)&WThi[lr][ks * 32 + 8 * lg];
                    const u32x4 awl = *(const u32x4 *)&WTlo[lr][ks * 32 + 8 * lg];
                    uint32_t kw[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t k0 = Ks[ks * 32 + 8 * lg + 2 * e][kc];
                        const uint32_t k1 = Ks[ks * 32 + 8 * lg + 2 * e + 1][kc];
                        kw[e] = k0 | (k1 << 16);
                    }
                    const u32x4 bk = {kw[0], kw[1], kw[2], kw[3]};
                    dS = mfma_bf16(awh, bk, dS);
                    dS = mfma_bf16(awl, bk, dS);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    Sreg[j][i] = fmaf(gC, Sreg[j][i], dS[i]);
            }
        }
        __syncthreads();
        stage_state();
    }

#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int vv = v0 + 4 * lg + i, kc = 16 * (2 * w + j) + lr;
            p.new_state[n * p.ns_sn + h * p.ns_sh + vv * p.ns_sv + kc] = Sreg[j][i];
        }
}

}  // namespace gdn

// ------------------------------------------------------------------------- host side
namespace {

constexpr int64_t kChunkH = 64;
constexpr int kZeroFillBlocks = 64;

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

int64_t max_chunks(int64_t T, int64_t N) { return (T + kChunkH - 1) / kChunkH + N; }

struct Layout {
    int64_t nc;
    int64_t header, chunk_tok0, chunk_len, seq_chunk0, seq_order, seq_tok0, seq_len, records,
        total;
};

Layout layout(int64_t T, int64_t N, int64_t HV)
{
    Layout L;
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
    L.seq_order = o;
    o += N * 4;
    L.seq_tok0 = o;
    o += N * 4;
    L.seq_len = o;
    o += N * 4;
    L.records = align256(o);
    L.total = L.records + L.nc * HV * gdn::kRecBytes;
    return L;
}

bool aligned(const void *p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

}  // namespace

extern "C" int64_t gdn_prefill_workspace_size(int32_t total_tokens, int32_t num_seqs,
                                              int32_t num_qk_heads, int32_t num_v_heads,
                                              int32_t head_size)
{
    if (total_tokens < 0 || num_seqs < 0 || num_qk_heads <= 0 || num_v_heads <= 0 ||
        num_v_heads % num_qk_heads != 0 || head_size != 128)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill_workspace_size: bad sizes T=%d N=%d "
                             "HQK=%d HV=%d D=%d", total_tokens, num_seqs, num_qk_heads,
                             num_v_heads, head_size);
    return layout(total_tokens, num_seqs, num_v_heads).total;
}

extern "C" int gdn_prefill_launch(const gdn_prefill_params *p, void *stream)
{
    if (!p || p->struct_size != (int32_t)sizeof(gdn_prefill_params))
        return gdn_set_error(GDN_EINVAL, "gdn_prefill: params NULL or struct_size mismatch");
    const int T = p->total_tokens, N = p->num_seqs, HQK = p->num_qk_heads,
              HV = p->num_v_heads, D = p->head_size;
    if (T < 0 || N < 0 || HQK <= 0 || HV <= 0 || HV % HQK != 0)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill: bad sizes T=%d N=%d HQK=%d HV=%d", T, N,
                             HQK, HV);
    if (D != 128)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill: head_size %d unsupported (128 only)", D);
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
    if (!aligned(p->q, 16) || !aligned(p->k, 16) || !aligned(p->output, 16))
        return gdn_set_error(GDN_ELAYOUT, "gdn_prefill: q/k/output must be 16-byte aligned");
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
    pa.seq_order = (int32_t *)(ws + L.seq_order);
    pa.seq_tok0 = (int32_t *)(ws + L.seq_tok0);
    pa.seq_len = (int32_t *)(ws + L.seq_len);
    pa.out = (gdn::bf16_t *)p->output;
    pa.o_st = p->output_stride[0];
    pa.o_sh = p->output_stride[1];
    hipLaunchKernelGGL(gdn::gdn_prefill_plan_kernel, dim3(1 + kZeroFillBlocks), dim3(256), 0,
                       st, pa);
    int rc = gdn_check_launch("gdn_prefill_plan_kernel");
    if (rc)
        return rc;

    if (L.nc > 0 && T > 0) {
        gdn::PrepArgs qa;
        qa.q = (const gdn::bf16_t *)p->q;
        qa.k = (const gdn::bf16_t *)p->k;
        qa.a = (const gdn::bf16_t *)p->a;
        qa.b = (const gdn::bf16_t *)p->b;
        qa.A_log = p->A_log;
        qa.dt_bias = p->dt_bias;
        qa.q_st = p->q_stride[0];
        qa.q_sh = p->q_stride[1];
        qa.k_st = p->k_stride[0];
        qa.k_sh = p->k_stride[1];
        qa.a_st = p->a_stride[0];
        qa.a_sh = p->a_stride[1];
        qa.b_st = p->b_stride[0];
        qa.b_sh = p->b_stride[1];
        qa.A_log_s = p->A_log_stride;
        qa.dt_s = p->dt_bias_stride;
        qa.header = pa.header;
        qa.chunk_tok0 = pa.chunk_tok0;
        qa.chunk_len = pa.chunk_len;
        qa.records = ws + L.records;
        qa.HV = HV;
        qa.ratio = ratio;
        if (L.nc > 0x7fffffff || HQK > 65535)
            return gdn_set_error(GDN_EINVAL, "gdn_prefill: grid too large");
        hipLaunchKernelGGL(gdn::gdn_prefill_prep_kernel, dim3((unsigned)L.nc, HQK), dim3(256), 0,
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
        sa.seq_order = pa.seq_order;
        sa.seq_tok0 = pa.seq_tok0;
        sa.seq_len = pa.seq_len;
        sa.records = ws + L.records;
        sa.HQK = HQK;
        sa.HV = HV;
        sa.ratio = ratio;
        sa.scale = p->scale;
        const int64_t ngroups = (int64_t)N * HQK;
        sa.ngroups = (int)ngroups;
        const int64_t blocks = 8 * (8 * (int64_t)ratio) * ((ngroups + 7) / 8);
        if (ngroups > 0x7fffffff || blocks > 0x7fffffff)
            return gdn_set_error(GDN_EINVAL, "gdn_prefill: grid too large");
        hipLaunchKernelGGL(gdn::gdn_prefill_scan_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                           sa);
        rc = gdn_check_launch("gdn_prefill_scan_kernel");
        if (rc)
            return rc;
    }
    return GDN_OK;
}
