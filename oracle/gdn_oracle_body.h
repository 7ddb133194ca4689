/*
 * Body of the CPU oracle, instantiated twice by gdn_oracle.c: once with
 * REAL = double (the float64 oracle, the parity target) and once with
 * REAL = float (a float32 restatement that follows the operation order of the
 * reference kernels, used to measure fp32 rounding noise).
 *
 * Requires the including file to define REAL, SFX (name suffix), and the math
 * functions EXP, LOG.
 *
 * Semantics (per v-head h, q/k head g = h / (HV/HQK), token t):
 *   x      = a[t,h] + dt_bias[h]                  gdn_decode/solution/triton/kernel.py:128
 *   sp     = x > 20 ? x : log(1 + exp(x))          gdn_decode/solution/triton/kernel.py:129
 *   alpha  = exp(-exp(A_log[h]) * sp)              gdn_decode/solution/triton/kernel.py:130
 *   beta   = 1 / (1 + exp(-b[t,h]))                gdn_decode/solution/triton/kernel.py:131
 *   old    = alpha * S                             gdn_decode/solution/triton/kernel.py:165
 *   u[v]   = sum_k old[v,k] * k[k]                 gdn_decode/solution/triton/kernel.py:166
 *   nv[v]  = beta * v[v] + (1 - beta) * u[v]       gdn_decode/solution/triton/kernel.py:167
 *   d[v]   = nv[v] - u[v]                          gdn_decode/solution/triton/kernel.py:168
 *   S[v,k] = old[v,k] + k[k] * d[v]                gdn_decode/solution/triton/kernel.py:169
 *   o[v]   = scale * sum_k S[v,k] * q[k]           gdn_decode/solution/triton/kernel.py:170,216
 * The state is k-last: S[v,k] lives at state[..., v, k]
 * (gdn_decode/solution/triton/kernel.py:8,17; gdn_prefill/solution/triton/kernel.py:32).
 */

#define CAT_(a, b) a##b
#define CAT(a, b) CAT_(a, b)

/* Gate scalars for one (token, v-head). */
static void CAT(gates_, SFX)(float A_log, float dt_bias, uint16_t a_bits, uint16_t b_bits,
                             REAL *alpha, REAL *beta)
{
    REAL x = (REAL)bf16_to_f32(a_bits) + (REAL)dt_bias;
    REAL sp = x > (REAL)20 ? x : LOG((REAL)1 + EXP(x));
    *alpha = EXP(-EXP((REAL)A_log) * sp);
    REAL bb = (REAL)bf16_to_f32(b_bits);
    *beta = (REAL)1 / ((REAL)1 + EXP(-bb));
}

/*
 * Run the recurrence for one (sequence, v-head) over tokens [t0, t1).
 * Token-indexed arrays are addressed as base + t * tok_stride + head * D.
 *   S        : D*D working state (k-last), updated in place
 *   q,k      : bf16 bits, token stride qk_tok (elements), head g
 *   v        : bf16 bits, token stride v_tok, head h
 *   a,b      : bf16 bits, token stride ab_tok, head h
 *   out      : REAL, token stride out_tok, head h (may be NULL)
 */
static void CAT(scan_head_, SFX)(int D, int t0, int t1, int g, int h,
                                 const uint16_t *q, const uint16_t *k, long qk_tok,
                                 const uint16_t *v, long v_tok,
                                 const uint16_t *a, const uint16_t *b, long ab_tok,
                                 float A_log, float dt_bias, REAL scale,
                                 REAL *S, REAL *out, long out_tok,
                                 REAL *kbuf, REAL *qbuf)
{
    for (int t = t0; t < t1; ++t) {
        REAL alpha, beta;
        CAT(gates_, SFX)(A_log, dt_bias, a[(long)t * ab_tok + h], b[(long)t * ab_tok + h],
                         &alpha, &beta);
        const uint16_t *qt = q + (long)t * qk_tok + (long)g * D;
        const uint16_t *kt = k + (long)t * qk_tok + (long)g * D;
        const uint16_t *vt = v + (long)t * v_tok + (long)h * D;
        for (int i = 0; i < D; ++i) {
            kbuf[i] = (REAL)bf16_to_f32(kt[i]);
            qbuf[i] = (REAL)bf16_to_f32(qt[i]);
        }
        for (int r = 0; r < D; ++r) {
            REAL *row = S + (long)r * D;
            REAL u = 0;
            for (int c = 0; c < D; ++c) {
                row[c] = alpha * row[c];
                u += row[c] * kbuf[c];
            }
            REAL nv = beta * (REAL)bf16_to_f32(vt[r]) + ((REAL)1 - beta) * u;
            REAL d = nv - u;
            REAL o = 0;
            for (int c = 0; c < D; ++c) {
                row[c] = row[c] + kbuf[c] * d;
                o += row[c] * qbuf[c];
            }
            if (out)
                out[(long)t * out_tok + (long)h * D + r] = scale * o;
        }
    }
}

/*
 * Decode: B sequences of one token each (seq_len = 1).
 * Shapes (contiguous): q,k [B,1,HQK,D]  v [B,1,HV,D]  state [B,HV,D,D] (NULL = zeros)
 * A_log, dt_bias [HV]  a,b [B,1,HV]  out [B,1,HV,D]  new_state [B,HV,D,D].
 * Follows gdn_decode/solution/triton/kernel.py:221-272 (host) and :71-218 (kernel).
 */
int CAT(oracle_decode_, SFX)(int B, int HQK, int HV, int D,
                             const uint16_t *q, const uint16_t *k, const uint16_t *v,
                             const float *state, const float *A_log, const uint16_t *a,
                             const float *dt_bias, const uint16_t *b, double scale,
                             REAL *out, REAL *new_state, int nthreads)
{
    if (B < 0 || HQK <= 0 || HV <= 0 || D <= 0 || HV % HQK != 0 || D > 512)
        return -1;
    const int ratio = HV / HQK;
    const long DD = (long)D * D;
    long npairs = (long)B * HV;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
    for (long p = 0; p < npairs; ++p) {
        int bi = (int)(p / HV), h = (int)(p % HV), g = h / ratio;
        REAL *S = new_state + p * DD;
        for (long i = 0; i < DD; ++i)
            S[i] = state ? (REAL)state[p * DD + i] : (REAL)0;
        REAL kbuf[512], qbuf[512];
        /* token index = bi, with every per-token array advanced by one batch row */
        CAT(scan_head_, SFX)(D, bi, bi + 1, g, h,
                             q, k, (long)HQK * D, v, (long)HV * D, a, b, (long)HV,
                             A_log[h], dt_bias[h], (REAL)scale,
                             S, out, (long)HV * D, kbuf, qbuf);
    }
    return 0;
}

/*
 * Prefill over packed variable-length sequences.
 * Shapes (contiguous): q,k [T,HQK,D]  v [T,HV,D]  a,b [T,HV]  cu_seqlens [N+1] (int64)
 * state [N,HV,D,D] (NULL = zeros)  out [T,HV,D]  new_state [N,HV,D,D].
 * Tokens outside every [cu[n], cu[n+1]) keep out = 0 (the reference zero-fills
 * output first: gdn_prefill/solution/triton/kernel.py:281-286).
 * Follows gdn_prefill/solution/triton/kernel.py:253-337 for the host contract and
 * the token recurrence above for the arithmetic.
 */
int CAT(oracle_prefill_, SFX)(int T, int N, int HQK, int HV, int D,
                              const uint16_t *q, const uint16_t *k, const uint16_t *v,
                              const float *state, const float *A_log, const uint16_t *a,
                              const float *dt_bias, const uint16_t *b,
                              const int64_t *cu_seqlens, double scale,
                              REAL *out, REAL *new_state, int nthreads)
{
    if (T < 0 || N < 0 || HQK <= 0 || HV <= 0 || D <= 0 || HV % HQK != 0 || D > 512)
        return -1;
    for (int n = 0; n < N; ++n)
        if (cu_seqlens[n] < 0 || cu_seqlens[n + 1] < cu_seqlens[n] || cu_seqlens[n + 1] > T)
            return -2;
    const int ratio = HV / HQK;
    const long DD = (long)D * D;
    for (long i = 0; i < (long)T * HV * D; ++i)
        out[i] = 0;
    long npairs = (long)N * HV;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
    for (long p = 0; p < npairs; ++p) {
        int n = (int)(p / HV), h = (int)(p % HV), g = h / ratio;
        REAL *S = new_state + p * DD;
        for (long i = 0; i < DD; ++i)
            S[i] = state ? (REAL)state[p * DD + i] : (REAL)0;
        REAL kbuf[512], qbuf[512];
        CAT(scan_head_, SFX)(D, (int)cu_seqlens[n], (int)cu_seqlens[n + 1], g, h,
                             q, k, (long)HQK * D, v, (long)HV * D, a, b, (long)HV,
                             A_log[h], dt_bias[h], (REAL)scale,
                             S, out, (long)HV * D, kbuf, qbuf);
    }
    return 0;
}

#undef CAT
#undef CAT_
