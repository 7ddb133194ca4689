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

constexpr int kC = 64;   // chunk length
constexpr int kDK = 128; // head size
constexpr int kLdK = 136; // padded LDS row (bf16) for 64 x 128 tiles
constexpr int kLdT = 72;  // padded LDS row (bf16) for 16 x 64 tiles

// Per (chunk, v-head) record in the workspace. 64x64 lower-triangular matrices are
// stored as their 10 lower 16x16 blocks, block (i, j <= i) at index i(i+1)/2 + j,
// each block row-major: exactly the rows and 8-column runs an MFMA A operand reads.
constexpr int kBlk = 256;        // elements per 16x16 block
constexpr int kRecThi = 0;       // bf16 [10][16][16]  T = (I + A)^-1, high half
constexpr int kRecTlo = 5120;    // bf16 [10][16][16]  low half
constexpr int kRecP = 10240;     // bf16 [10][16][16]  P (decayed, causal Q K^T)
constexpr int kRecGates = 15360; // f32 beta[64], gamma[64], dec[64], gammaC
constexpr int kRecZero = 16256;  // 16 zero bytes (after the gates): what absent blocks read
constexpr int kRecBytes = 16384;

__device__ __forceinline__ int tri_blk(int i, int j) { return i * (i + 1) / 2 + j; }

// Workgroup barrier that orders LDS only: global loads issued before it (the next
// chunk's prefetch) stay in flight across it.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int K>
__device__ __forceinline__ float quad_bcast(float x)
{
    return dpp_mov<K | (K << 2) | (K << 4) | (K << 6)>(x);
}

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
    int HQK, HV, ratio;
};

// Lower-triangular 16x16 tile t of a 64x64 matrix -> (row block, column block).
__device__ __forceinline__ int tile_i(int t) { return t < 1 ? 0 : (t < 3 ? 1 : (t < 6 ? 2 : 3)); }
__device__ __forceinline__ int tile_j(int t) { return t - tri_blk(tile_i(t), 0); }

__device__ __forceinline__ float quad_bcast_sel(float x, int k)
{
    switch (k & 3) {
    case 0: return quad_bcast<0>(x);
    case 1: return quad_bcast<1>(x);
    case 2: return quad_bcast<2>(x);
    default: return quad_bcast<3>(x);
    }
}

__global__ __launch_bounds__(256) void gdn_prefill_prep_kernel(PrepArgs p)
{
    // One workgroup per (chunk, v-head). The `ratio` v-heads of one (chunk, q/k head)
    // read the same K and Q: their workgroups land on one XCD (ids are dealt to the 8
    // XCDs round-robin), so the second read hits that XCD's L2.
    const int pid = blockIdx.x, xcd = pid & 7, slot = pid >> 3;
    const int hh = slot % p.ratio;
    const int grp = (slot / p.ratio) * 8 + xcd;
    const int c = grp / p.HQK, g = grp % p.HQK;
    if (c >= p.header[0])
        return;
    const int h = g * p.ratio + hh;
    const int tok0 = p.chunk_tok0[c];
    const int len = p.chunk_len[c];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lr = l & 15, lg = l >> 4;

    // K and Q (bf16) first; the same bytes then hold A and T (fp32).
    __shared__ __align__(16) char smem[2 * kC * kLdK * 2];
    __shared__ __align__(16) bf16_t Ps[10 * kBlk];
    __shared__ __align__(16) float Ms[4][16][17];
    __shared__ float Lg[kC], Bt[kC];
    bf16_t(*Ks)[kLdK] = (bf16_t(*)[kLdK])smem;
    bf16_t(*Qs)[kLdK] = (bf16_t(*)[kLdK])(smem + kC * kLdK * 2);
    float(*As)[kC + 4] = (float(*)[kC + 4])smem;
    float(*Ts)[kC + 4] = (float(*)[kC + 4])(smem + kC * (kC + 4) * 4);
    static_assert(2 * kC * (kC + 4) * 4 == 2 * kC * kLdK * 2, "A/T alias K/Q exactly");

    char *rec = p.records + ((int64_t)c * p.HV + h) * kRecBytes;

    // Wave 0's gate inputs (one token per lane) are requested first, then K and Q.
    uint32_t a_raw = 0u, b_raw = 0u;
    if (w == 0) {
        const int t = tok0 + min(l, len - 1);
        a_raw = p.a[(int64_t)t * p.a_st + h * p.a_sh];
        b_raw = p.b[(int64_t)t * p.b_st + h * p.b_sh];
    }
    // K, Q chunk rows -> LDS. All eight 16-byte loads per lane are issued before the
    // first store. Rows past the chunk's end repeat its last token: they only meet
    // beta = 0 (in A) or the causal mask (in P), so they contribute nothing.
    {
        u32x4 kv[4], qv[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int s = tid + 256 * m, row = min(s >> 4, len - 1), col = (s & 15) * 8;
            kv[m] = *(const u32x4 *)(p.k + (int64_t)(tok0 + row) * p.k_st + g * p.k_sh + col);
            qv[m] = *(const u32x4 *)(p.q + (int64_t)(tok0 + row) * p.q_st + g * p.q_sh + col);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int s = tid + 256 * m, row = s >> 4, col = (s & 15) * 8;
            *(u32x4 *)&Ks[row][col] = kv[m];
            *(u32x4 *)&Qs[row][col] = qv[m];
        }
    }

    // Gates and in-chunk cumulative log decay: wave 0, one lane per token
    // (gdn_decode/solution/triton/kernel.py:128-131). Padding tokens: alpha = 1, beta = 0.
    if (w == 0) {
        float la = 0.f, bt = 0.f;
        if (l < len) {
            const float x = bf16_to_f32(a_raw) + p.dt_bias[h * p.dt_s];
            const float sp = x > 20.f ? x : logf(1.f + expf(x));
            la = -expf(p.A_log[h * p.A_log_s]) * sp;
            bt = 1.f / (1.f + expf(-bf16_to_f32(b_raw)));
        }
        // cumulative decay in log2 units: every decay factor below is 2^(non-positive
        // difference), one v_exp_f32 (results below 2^-126 flush to 0, i.e. underflow)
        float L = la * 1.44269504088896340736f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float y = __shfl_up(L, off, 64);
            if (l >= off)
                L += y;
        }
        const float Lend = __shfl(L, 63, 64);
        Lg[l] = L;
        Bt[l] = bt;
        float *gates = (float *)(rec + kRecGates);
        gates[l] = bt;
        gates[64 + l] = __builtin_amdgcn_exp2f(L);
        gates[128 + l] = __builtin_amdgcn_exp2f(Lend - L);
        if (l == 0)
            gates[192] = __builtin_amdgcn_exp2f(Lend);
        if (l < 4)
            ((float *)(rec + kRecZero))[l] = 0.f;
    }
    lds_barrier();

    // 20 tile jobs (10 lower tiles of K K^T, 10 of Q K^T), 5 per wave.
    f32x4 acc[5];
#pragma unroll
    for (int m = 0; m < 5; ++m) {
        const int job = w + 4 * m;
        const bool isq = job >= 10;
        const int t = isq ? job - 10 : job;
        const int ti = tile_i(t), tj = tile_j(t);
        f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const u32x4 a = isq ? *(const u32x4 *)&Qs[16 * ti + lr][ks * 32 + 8 * lg]
                                : *(const u32x4 *)&Ks[16 * ti + lr][ks * 32 + 8 * lg];
            const u32x4 bk = *(const u32x4 *)&Ks[16 * tj + lr][ks * 32 + 8 * lg];
            r = mfma_bf16(a, bk, r);
        }
        acc[m] = r;
        if (isq) {  // P = exp(L_t - L_j) q_t . k_j for j <= t, bf16, block layout
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int tt = 16 * ti + 4 * lg + e, jj = 16 * tj + lr;
                const float pv = jj <= tt ? __builtin_amdgcn_exp2f(Lg[tt] - Lg[jj]) * r[e] : 0.f;
                Ps[t * kBlk + (4 * lg + e) * 16 + lr] = (bf16_t)f32_to_bf16(pv);
            }
        }
    }
    lds_barrier();  // K and Q are no longer read: their bytes become A and T

    // A[t,j] = beta_t exp(L_t - L_j) k_t . k_j, j < t
#pragma unroll
    for (int m = 0; m < 5; ++m) {
        const int job = w + 4 * m;
        if (job < 10) {
            const int ti = tile_i(job), tj = tile_j(job);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int tt = 16 * ti + 4 * lg + e, jj = 16 * tj + lr;
                As[tt][jj] = jj < tt ? Bt[tt] * __builtin_amdgcn_exp2f(Lg[tt] - Lg[jj]) * acc[m][e] : 0.f;
            }
        }
    }
    for (int q = tid; q < 10 * kBlk / 8; q += 256)
        *(u32x4 *)(rec + kRecP + q * 16) = *(const u32x4 *)((const char *)Ps + q * 16);
    lds_barrier();

    // Diagonal blocks of T = (I + A)^-1: wave i inverts block i by right-looking
    // substitution; lane = 4 * column + row group, each lane holding rows g4 + 4m.
    {
        const int o = 16 * w, col = l >> 2, g4 = l & 3;
        float x[4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
            x[m] = (g4 + 4 * m == col) ? 1.f : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float xr = quad_bcast_sel(x[r >> 2], r & 3);  // final x_r of this column
#pragma unroll
            for (int m = 0; m < 4; ++m)  // A is zero on and above the diagonal
                x[m] = fmaf(-As[o + g4 + 4 * m][o + r], xr, x[m]);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m)
            Ts[o + g4 + 4 * m][o + col] = x[m];
    }
    lds_barrier();

    // Off-diagonal blocks, one block diagonal at a time (fp32 MFMA 16x16x4):
    //   T_ij = -T_ii * sum_{m=j}^{i-1} A_im T_mj
    for (int d = 1; d < 4; ++d) {
        const int i = w + d, j = w;
        const bool active = i < 4;
        if (active) {
            f32x4 M = {0.f, 0.f, 0.f, 0.f};
            for (int m = j; m < i; ++m) {
#pragma unroll
                for (int k4 = 0; k4 < 4; ++k4)
                    M = mfma_f32(As[16 * i + lr][16 * m + 4 * k4 + lg],
                                 Ts[16 * m + 4 * k4 + lg][16 * j + lr], M);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                Ms[w][4 * lg + e][lr] = M[e];
        }
        lds_barrier();
        if (active) {
            f32x4 R = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k4 = 0; k4 < 4; ++k4)
                R = mfma_f32(Ts[16 * i + lr][16 * i + 4 * k4 + lg], Ms[w][4 * k4 + lg][lr], R);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                Ts[16 * i + 4 * lg + e][16 * j + lr] = -R[e];
        }
        lds_barrier();
    }

    // T -> record (bf16 hi / lo, block layout); 16-byte pieces.
    for (int q = tid; q < 10 * kBlk / 8; q += 256) {
        const int bidx = q >> 5, row = (q & 31) >> 1, c8 = (q & 1) * 8;
        const int bi = tile_i(bidx), bj = tile_j(bidx);
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            split_bf16x2(Ts[16 * bi + row][16 * bj + c8 + 2 * e],
                         Ts[16 * bi + row][16 * bj + c8 + 2 * e + 1], hw[e], lw[e]);
        *(u32x4 *)(rec + kRecThi + q * 16) = u32x4{hw[0], hw[1], hw[2], hw[3]};
        *(u32x4 *)(rec + kRecTlo + q * 16) = u32x4{lw[0], lw[1], lw[2], lw[3]};
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

// One chunk's operands for one lane, loaded a chunk ahead (MFMA A-operand layouts).
struct ChunkRegs {
    u32x4 kf[4];         // K rows 16w+lr, columns 32ks + 8lg .. +7
    u32x4 th[2], tl[2];  // T hi / lo rows 16w+lr, columns 32ks + 8lg .. +7
    u32x4 pf[2];         // P, same layout as T
    uint32_t vv[4];      // V[16w + 4lg + i][v0 + lr] (bf16 bits)
    f32x4 beta, gamma, dec;  // gates of tokens 16w + 4lg + 0..3
    float gC;
};

// PREFETCH: the next chunk's operands are loaded into registers while the current
// chunk computes (two register sets, 2 waves per SIMD). Otherwise each chunk's
// loads are issued together at the start of its step (one set, more waves per SIMD
// hide the latency instead).
template <bool PREFETCH>
__device__ __forceinline__ void scan_body(const ScanArgs &p)
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

    // Addressing: per chunk a wave-uniform 64-bit base (scalar registers) plus a 32-bit
    // per-lane byte offset (the host keeps token / head strides below 2^24 elements),
    // so loads and stores use the scalar-base + vector-offset form.
    const int trow = 16 * w + lr;             // token row of this lane's A operands
    const int tcol = 16 * w + 4 * lg;         // first of this lane's 4 C-layout token rows
    const uint32_t kst2 = (uint32_t)p.k_st * 2, qst2 = (uint32_t)p.q_st * 2;
    const uint32_t vst2 = (uint32_t)p.v_st * 2, ost2 = (uint32_t)p.o_st * 2;
    const char *kbase = (const char *)(p.k + (int64_t)tok0 * p.k_st + g * p.k_sh);
    const char *qbase = (const char *)(p.q + (int64_t)tok0 * p.q_st + g * p.q_sh);
    const char *vbase = (const char *)(p.v + (int64_t)tok0 * p.v_st + h * p.v_sh);
    char *obase = (char *)(p.out + (int64_t)tok0 * p.o_st + h * p.o_sh);
    const int64_t kstep = (int64_t)kC * p.k_st * 2, qstep = (int64_t)kC * p.q_st * 2;
    const int64_t vstep = (int64_t)kC * p.v_st * 2, ostep = (int64_t)kC * p.o_st * 2;
    const char *rbase = p.records + ((int64_t)c0 * p.HV + h) * kRecBytes;
    const int64_t rstep = (int64_t)p.HV * kRecBytes;
    // Byte offsets of this lane's T / P A-operand pieces inside a record; blocks above
    // the diagonal are not stored and read the record's zero bytes instead.
    uint32_t thoff[2], tloff[2], poff[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int jb = 2 * ks + (lg >> 1);
        const uint32_t o = 2u * (tri_blk(w, jb) * kBlk + lr * 16 + 8 * (lg & 1));
        thoff[ks] = jb <= w ? kRecThi + o : kRecZero;
        tloff[ks] = jb <= w ? kRecTlo + o : kRecZero;
        poff[ks] = jb <= w ? kRecP + o : kRecZero;
    }
    const uint32_t lane_col = 16u * lg;                 // 8 bf16 per lane group
    const uint32_t v_col = 2u * (v0 + lr);
    const uint32_t o_col = 2u * (v0 + (lr & ~1));
    const uint32_t g_off = 4u * tcol;

    // Rows past a chunk's end are clamped to its last token instead of zeroed: they
    // carry beta = 0 and decay weight 0, so they contribute exactly nothing, and their
    // outputs are not stored. Every load reads valid memory and stays in flight.
    auto load_chunk = [&](ChunkRegs &r, int c) {
        const int lenc = min(kC, len - c * kC);
        const char *rec = rbase + c * rstep;
        const char *kc_ = kbase + c * kstep;
        const uint32_t ko = (uint32_t)min(trow, lenc - 1) * kst2 + lane_col;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            r.kf[ks] = *(const u32x4 *)(kc_ + ko + 64 * ks);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            r.th[ks] = *(const u32x4 *)(rec + thoff[ks]);
            r.tl[ks] = *(const u32x4 *)(rec + tloff[ks]);
            r.pf[ks] = *(const u32x4 *)(rec + poff[ks]);
        }
        const char *vc_ = vbase + c * vstep;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r.vv[i] = *(const bf16_t *)(vc_ + (uint32_t)min(tcol + i, lenc - 1) * vst2 + v_col);
        const char *gt = rec + kRecGates;
        r.beta = *(const f32x4 *)(gt + g_off);
        r.gamma = *(const f32x4 *)(gt + 256 + g_off);
        r.dec = *(const f32x4 *)(gt + 512 + g_off);
        r.gC = *(const float *)(gt + 768);
    };

    // State tile rows v0..v0+15 in MFMA C layout: Sreg[j][i] = S[v0 + 4 lg + i][16 (2w + j) + lr].
    f32x4 Sreg[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int vv = v0 + 4 * lg + i, kc = 16 * (2 * w + j) + lr;
            Sreg[j][i] = p.state ? p.state[n * p.st_sn + h * p.st_sh + vv * p.st_sv + kc] : 0.f;
        }
    // S -> LDS as bf16 hi / lo. Lanes lr and lr^1 hold neighbouring columns: even lanes
    // store rows 0,1 and odd lanes rows 2,3 of the pair as packed 32-bit words (element
    // indices stay static: the lane choice only predicates the stores).
    const bool even = (lr & 1) == 0;
    auto stage_state = [&]() {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = (16 * (2 * w + j) + lr) & ~1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float mine = Sreg[j][i];
                const float oth = dpp_mov<kDppQuadXor1>(mine);
                uint32_t hi, lo;
                split_bf16x2(even ? mine : oth, even ? oth : mine, hi, lo);
                if (even == (i < 2)) {
                    *(uint32_t *)&Shi[4 * lg + i][col] = hi;
                    *(uint32_t *)&Slo[4 * lg + i][col] = lo;
                }
            }
        }
    };
    stage_state();

    auto step = [&](ChunkRegs &cur, ChunkRegs &nxt, int c) {
        const int lenc = min(kC, len - c * kC);
        if constexpr (PREFETCH) {
            if (c + 1 < nck)
                load_chunk(nxt, c + 1);  // in flight while this chunk computes
        } else {
            load_chunk(cur, c);
        }
        // Q of this chunk: first needed by the readout (d), after three phases
        u32x4 qf[4];
        {
            const char *qc_ = qbase + c * qstep;
            const uint32_t qo = (uint32_t)min(trow, lenc - 1) * qst2 + lane_col;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                qf[ks] = *(const u32x4 *)(qc_ + qo + 64 * ks);
        }

        // K rows of this wave -> LDS (the state update reads K by columns)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            *(u32x4 *)&Ks[trow][ks * 32 + 8 * lg] = cur.kf[ks];
        lds_barrier();

        // (a) X = K S0^T for tokens 16w..16w+15 (S0 as hi + lo; two accumulators keep
        // the dependent MFMA chains short)
        f32x4 X = {0.f, 0.f, 0.f, 0.f}, Xl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const u32x4 bh = *(const u32x4 *)&Shi[lr][ks * 32 + 8 * lg];
            const u32x4 bl = *(const u32x4 *)&Slo[lr][ks * 32 + 8 * lg];
            X = mfma_bf16(cur.kf[ks], bh, X);
            Xl = mfma_bf16(cur.kf[ks], bl, Xl);
        }
        X += Xl;
        // (b) R = beta (V - gamma X) -> LDS as R^T (hi, lo)
        {
            float r[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                r[i] = cur.beta[i] * (bf16_to_f32(cur.vv[i]) - cur.gamma[i] * X[i]);
            uint32_t h01, l01, h23, l23;
            split_bf16x2(r[0], r[1], h01, l01);
            split_bf16x2(r[2], r[3], h23, l23);
            *(u32x2 *)&RThi[lr][tcol] = u32x2{h01, h23};
            *(u32x2 *)&RTlo[lr][tcol] = u32x2{l01, l23};
        }
        lds_barrier();

        // (c) U = T R  (T, R as hi + lo; three products). Rows < 32 of T have no
        // entries in columns >= 32.
        f32x4 U = {0.f, 0.f, 0.f, 0.f}, Ul = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            if (ks == 1 && w < 2)
                continue;
            const u32x4 bh = *(const u32x4 *)&RThi[lr][ks * 32 + 8 * lg];
            const u32x4 bl = *(const u32x4 *)&RTlo[lr][ks * 32 + 8 * lg];
            U = mfma_bf16(cur.th[ks], bh, U);
            Ul = mfma_bf16(cur.th[ks], bl, Ul);
            Ul = mfma_bf16(cur.tl[ks], bh, Ul);
        }
        U += Ul;
        {
            uint32_t wh01, wl01, wh23, wl23;
            split_bf16x2(cur.dec[0] * U[0], cur.dec[1] * U[1], wh01, wl01);
            split_bf16x2(cur.dec[2] * U[2], cur.dec[3] * U[3], wh23, wl23);
            *(u32x2 *)&UThi[lr][tcol] = u32x2{pack_bf16x2(U[0], U[1]), pack_bf16x2(U[2], U[3])};
            *(u32x2 *)&WThi[lr][tcol] = u32x2{wh01, wh23};
            *(u32x2 *)&WTlo[lr][tcol] = u32x2{wl01, wl23};
        }
        lds_barrier();

        // (d) O = scale (gamma Q S0^T + P U) for tokens 16w..16w+15
        {
            f32x4 Oi = {0.f, 0.f, 0.f, 0.f}, Oa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                Oi = mfma_bf16(qf[ks], *(const u32x4 *)&Shi[lr][ks * 32 + 8 * lg], Oi);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                if (ks == 1 && w < 2)
                    continue;
                Oa = mfma_bf16(cur.pf[ks], *(const u32x4 *)&UThi[lr][ks * 32 + 8 * lg], Oa);
            }
            // lanes lr, lr^1 pack neighbouring columns: even lanes store rows 0,1, odd 2,3
            char *oc_ = obase + c * ostep;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float mine = p.scale * fmaf(cur.gamma[i], Oi[i], Oa[i]);
                const float oth = dpp_mov<kDppQuadXor1>(mine);
                const uint32_t packed = pack_bf16x2(even ? mine : oth, even ? oth : mine);
                if (even == (i < 2) && tcol + i < lenc)
                    *(uint32_t *)(oc_ + (uint32_t)(tcol + i) * ost2 + o_col) = packed;
            }
        }

        // (e) S = gammaC S + W^T K over this wave's 32 state columns
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int kc = 16 * (2 * w + j) + lr;
            f32x4 dS = {0.f, 0.f, 0.f, 0.f}, dSl = {0.f, 0.f, 0.f, 0.f};
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
                dSl = mfma_bf16(awl, bk, dSl);
            }
            dS += dSl;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                Sreg[j][i] = fmaf(cur.gC, Sreg[j][i], dS[i]);
        }
        lds_barrier();
        stage_state();
    };

    if constexpr (PREFETCH) {
        ChunkRegs ra, rb;
        if (nck > 0)
            load_chunk(ra, 0);
        for (int c = 0; c < nck; c += 2) {
            step(ra, rb, c);
            if (c + 1 < nck)
                step(rb, ra, c + 1);
        }
    } else {
        ChunkRegs r;
        for (int c = 0; c < nck; ++c)
            step(r, r, c);
    }

#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int vv = v0 + 4 * lg + i, kc = 16 * (2 * w + j) + lr;
            p.new_state[n * p.ns_sn + h * p.ns_sh + vv * p.ns_sv + kc] = Sreg[j][i];
        }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
gdn_prefill_scan_kernel(ScanArgs p)
{
    scan_body<true>(p);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void
gdn_prefill_scan_kernel_nopf3(ScanArgs p)
{
    scan_body<false>(p);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void
gdn_prefill_scan_kernel_nopf4(ScanArgs p)
{
    scan_body<false>(p);
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
    // the kernels address a 64-token chunk with 32-bit byte offsets
    const int64_t kMaxStride = int64_t(1) << 24;
    for (int i = 0; i < 2; ++i)
        if (p->q_stride[i] >= kMaxStride || p->k_stride[i] >= kMaxStride ||
            p->v_stride[i] >= kMaxStride || p->output_stride[i] >= kMaxStride ||
            p->q_stride[i] < 0 || p->k_stride[i] < 0 || p->v_stride[i] < 0 ||
            p->output_stride[i] < 0)
            return gdn_set_error(GDN_ELAYOUT,
                                 "gdn_prefill: token / head strides must be in [0, 2^24)");
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
        qa.HQK = HQK;
        qa.HV = HV;
        qa.ratio = ratio;
        const int64_t units = L.nc * HQK;  // (chunk, q/k head) groups
        const int64_t blocks = 8 * (int64_t)ratio * ((units + 7) / 8);
        if (blocks > 0x7fffffff)
            return gdn_set_error(GDN_EINVAL, "gdn_prefill: grid too large");
        hipLaunchKernelGGL(gdn::gdn_prefill_prep_kernel, dim3((unsigned)blocks), dim3(256), 0,
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
        // variant (tuning sweeps): 0 = per-chunk batched loads at 3 waves per SIMD (the
        // fastest on MI355X), 1 = next-chunk register prefetch at 2 waves per SIMD,
        // 2 = batched loads at 4 waves per SIMD
        if (p->variant == 1)
            hipLaunchKernelGGL(gdn::gdn_prefill_scan_kernel, dim3((unsigned)blocks), dim3(256),
                               0, st, sa);
        else if (p->variant == 2)
            hipLaunchKernelGGL(gdn::gdn_prefill_scan_kernel_nopf4, dim3((unsigned)blocks),
                               dim3(256), 0, st, sa);
        else
            hipLaunchKernelGGL(gdn::gdn_prefill_scan_kernel_nopf3, dim3((unsigned)blocks),
                               dim3(256), 0, st, sa);
        rc = gdn_check_launch("gdn_prefill_scan_kernel");
        if (rc)
            return rc;
    }
    return GDN_OK;
}
