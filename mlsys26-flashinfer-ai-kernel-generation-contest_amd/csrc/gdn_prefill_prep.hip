// Prefill prep kernels: per (chunk, q/k head, v-head pair) unit, gates, P' and
// T' = (I + A)^-1 diag(beta) into the chunk's records.
#include "gdn_prefill.h"

namespace gdn {

// Work unit: (chunk, q/k head, group of VH v-heads). A persistent workgroup of 4 VH waves
// walks units u = blockIdx.x, + gridDim.x, ...; wave (hv, w) = v-head hv of the group,
// block w. The unit's K and Q go to LDS once (direct copies; K double-buffered, the next
// unit's copies and gate inputs in flight while this one computes) and serve every
// v-head of the group. Per unit, wave (hv, w):
//   * writes P' row block w: P'[t, j] = scale 2^(L_t - L_j) q_t . k_j, j <= t;
//   * forms A column block w, A[t, j] = beta_t 2^(L_t - L_j) k_t . k_j (j < t): the
//     diagonal block stays in registers, blocks (i > w, w) go to LDS for every wave;
//   * inverts X_w = (I + A_ww)^-1 by forward substitution (DPP broadcasts);
//   * after a barrier (all X_i and A blocks published): column block w of T = (I + A)^-1,
//       T_ww = X_w,  T_iw = -X_i sum_{m=w}^{i-1} A_im T_mw  (i > w),
//     on fp32 MFMA with every operand in registers, and writes T' = T diag(beta);
// (T', P' and dec are stored in the similarity form given with the gates below)
// wave (hv, 3), which has the least work after the barrier, also computes the next unit's
// gates and cumulative log2 decay L.
// (gdn_prefill/solution/triton/kernel.py:60-79 form the same A, T and P.)
// K and Q rows in LDS: row t, k-chunk c (k = 8c .. 8c + 7) at unit 16 t + (c ^ pswz(t & 15)).
// The MFMA operand reads take rows in token order (P' blocks) and in the pi order of the
// A blocks; with the plain XOR (c ^ t) the pi-ordered reads were 2-way bank conflicts, as
// both 16-lane groups of a read cycle hit the same eight units. Flipping bit 1 with bit 0
// of the row makes both orders conflict-free under the b128 bank model (one cycle: a
// 32-lane half with equal parity of lane bits 2, 3, 4; 16 distinct units mod 256 bytes).
__device__ __forceinline__ int pswz(int r) { return r ^ ((r & 1) << 1); }

template <int VH>
struct PrepSmem {
    u32x4 K[2][kC * 16];  // row t, k-chunk c at unit 16 t + (c ^ pswz(t & 15))
    u32x4 Q[kC * 16];
    float L[2][VH][64];    // L by token: L = L_hi + L_lo (float-float), L_hi here
    float Llo[2][VH][64];  // L_lo by token
    float B[2][VH][64];   // beta by token
    u32x4 XA[VH][4][64];  // X_w in A-operand layout, by lane, split4
    u32x4 AO[VH][6][64];  // off-diagonal A_im (m < i) as XA; index i(i-1)/2 + m
    float Ms[4 * VH][16][16];  // per wave: -A_ww rows, X_w, then T' staging
    // self-planned launches: sequence n's first chunk (clamped to nc; nc past the N
    // sequences), first token and length; the chunk total and the covered tokens [g0, g1)
    int32_t s_first[kSelfPlanMax], s_t0[kSelfPlanMax], s_len[kSelfPlanMax];
    int32_t s_total, s_g0, s_g1, s_pad;
};

constexpr int kGateWave = 3;  // column block with no work after the barrier

// Self-planned launch: wave 0 of every workgroup builds the sequence table in LDS from
// cu_seqlens, with the plan kernel's clamps (gdn_prefill_plan.hip), so both give the same
// chunk numbering; the last block, which walks the fewest units, then writes what the scan
// reads (sequence tables, longest-first order, chunk total, segment jobs) and every
// workgroup zero-fills its share of the output rows outside [cu[0], cu[N]).
template <int VH>
__device__ __forceinline__ void self_plan(const PrepArgs &p, PrepSmem<VH> &sm, int wv, int l)
{
    const PlanArgs &q = p.plan;
    if (wv == 0) {
        int t0 = 0, ln = 0;
        int64_t nck = 0, braw = 0;
        if (l < q.N) {
            int64_t a = load_cu(q.cu, q.cu64, l), b = load_cu(q.cu, q.cu64, l + 1);
            braw = b;
            a = a < 0 ? 0 : (a > q.T ? q.T : a);
            b = b < a ? a : (b > q.T ? q.T : b);
            t0 = (int)a;
            ln = (int)(b - a);
            nck = (ln + kC - 1) / kC;
        }
        const int64_t incl = wave_prefix_sum_i64(nck), first = incl - nck;
        sm.s_first[l] = l < q.N ? (int32_t)(first < q.nc ? first : q.nc) : q.nc;
        sm.s_t0[l] = t0;
        sm.s_len[l] = ln;
        if (l == 63)
            sm.s_total = (int32_t)(incl < q.nc ? incl : q.nc);
        // Cross-lane reads stay in wave-uniform control flow: inside a lane-conditional
        // branch the compiler may reuse the source register in lanes outside the branch.
        const int last = q.N - 1;
        const int64_t b_hi = __builtin_amdgcn_readlane((int)(braw >> 32), last),
                      b_lo = (uint32_t)__builtin_amdgcn_readlane((int)braw, last);
        const int64_t g1 = (b_hi << 32) | b_lo;
        const int g0 = __builtin_amdgcn_readlane(t0, 0);  // cu[0] clamped to [0, T]
        if (l == 0) {
            sm.s_g0 = g0;
            sm.s_g1 = (int32_t)(g1 < g0 ? g0 : (g1 > q.T ? q.T : g1));
        }
    }
    __syncthreads();
    if (blockIdx.x == gridDim.x - 1 && wv == 0) {
        const int first = sm.s_first[l], t0 = sm.s_t0[l], ln = sm.s_len[l];
        const int nck = (ln + kC - 1) / kC;
        int rank = 0;
        for (int m = 0; m < q.N; ++m) {
            const int o = __builtin_amdgcn_readlane(nck, m);
            rank += (o > nck) || (o == nck && m < l);
        }
        // the second K buffer is not written before the first unit's barrier
        int32_t *order = (int32_t *)sm.K[1];
        if (l < q.N) {
            q.seq_tok0[l] = t0;
            q.seq_len[l] = ln;
            q.seq_chunk0[l] = first;
            *(int4 *)(q.seq_rank + 4 * rank) = int4{l, t0, ln, first};
            order[rank] = l;
        }
        if (l == 0) {
            q.seq_chunk0[q.N] = sm.s_total;
            q.header[0] = sm.s_total;
        }
        if (q.seg_G >= 3)  // every lane of the wave takes part
            plan_jobs(q, order, sm.s_first, sm.s_t0, sm.s_len, l);
        if (q.whole_cus > 0) {
            // Whole sequences, both scans launched. The 4-wave scan spreads each (sequence,
            // v-head) over two CUs: a chunk takes ~0.74 of the 8-wave scan's time, but
            // costs 1.5 times the CU time. It is the faster while its average load per CU
            // (chunk-times over all jobs) stays below the longest sequence, which bounds
            // both scans from below (measured on MI355X at load / longest: 0.71 -13 %,
            // 1.02 -4 %, 1.06 +3 %, 1.27 +6 %); 0.9 leaves the close calls to the 8-wave
            // scan.
            const float cmax = wave_max_nonneg((float)nck);
            const float load4 = 2.f * (float)sm.s_total * (float)q.HO / (float)q.whole_cus;
            const bool use4 = load4 <= 0.9f * cmax;
            if (l == 0) {
                q.header[4] = use4 ? q.N : 0;
                q.header[5] = use4 ? 0 : q.N;
            }
        }
    }
    const int g0 = sm.s_g0, g1 = sm.s_g1, gap = g0 + (q.T - g1);
    if (gap > 0) {
        const int per_tok = q.HO * (kDK / 8);
        const u32x4 z = {0u, 0u, 0u, 0u};
        for (int gt = blockIdx.x; gt < gap; gt += gridDim.x) {
            const int64_t tok = gt < g0 ? gt : g1 + (gt - g0);
            for (int v = threadIdx.x; v < per_tok; v += blockDim.x)
                *(u32x4 *)(q.out + tok * q.o_st + (v >> 4) * q.o_sh + (v & 15) * 8) = z;
        }
    }
}

template <int VH>
__device__ __forceinline__ void prep_body(const PrepArgs &p, PrepSmem<VH> &sm)
{
    const int ngrp = p.ratio / VH;
    // wv is wave-uniform: branches on the column block are scalar branches
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63,
              lr = l & 15, lg = l >> 4;
    if (p.self_plan)
        self_plan(p, sm, wv, l);
    // (values read from LDS are uniform here; readfirstlane tells the compiler so, or every
    // branch on them would become a divergent one)
    const int nunits =
        (p.self_plan ? __builtin_amdgcn_readfirstlane(sm.s_total) : p.header[0]) * p.HQK * ngrp;
    // Waves are dealt to the 4 SIMDs round-robin: the second v-head takes the blocks in
    // reverse, so each SIMD pairs a heavy column block (w = 0) with a light one.
    const int hv = wv >> 2, w = hv & 1 ? 3 - (wv & 3) : (wv & 3);
    const uint32_t kst2 = (uint32_t)p.k_st * 2, qst2 = (uint32_t)p.q_st * 2;

    struct Unit {
        int c, g, h, tok0, len;
    };
    auto unit = [&](int u) {
        Unit r;
        const int grp = u / ngrp, hg = u % ngrp;
        r.c = grp / p.HQK;
        r.g = grp % p.HQK;
        r.h = r.g * p.ratio + hg * VH + hv;
        if (p.self_plan) {
            // the owner of chunk c is the last sequence whose first chunk is <= c (first
            // chunks never decrease; an empty sequence shares its successor's first chunk)
            const int f = sm.s_first[l];
            const int n = __popcll(__ballot(f <= r.c)) - 1;
            const int i = r.c - __builtin_amdgcn_readlane(f, n);
            r.tok0 = __builtin_amdgcn_readfirstlane(sm.s_t0[n]) + kC * i;
            r.len = min(kC, __builtin_amdgcn_readfirstlane(sm.s_len[n]) - kC * i);
        } else {
            r.tok0 = p.chunk_tok0[r.c];
            r.len = p.chunk_len[r.c];
        }
        return r;
    };
    // K or Q of a unit -> LDS: 16 windows of 64 16-byte units (4 rows each) per matrix,
    // dealt to the waves. Rows past the chunk's end repeat its last token: they meet
    // beta = 0 or the causal mask only.
    auto copy = [&](const Unit &U, bool isq, u32x4 *dst) {
        const char *base = isq ? (const char *)(p.q + (int64_t)U.tok0 * p.q_st + (int64_t)U.g * p.q_sh)
                               : (const char *)(p.k + (int64_t)U.tok0 * p.k_st + (int64_t)U.g * p.k_sh);
        const uint32_t st2 = isq ? qst2 : kst2;
#pragma unroll
        for (int i = 0; i < 4 / VH; ++i) {
            const int b = wv + 4 * VH * i;
            const int t = 4 * b + (l >> 4), cs = l & 15;
            dma16(base + (uint32_t)min(t, U.len - 1) * st2 + 16u * (cs ^ pswz(t & 15)),
                  &dst[64 * b]);
        }
    };
    // Gates (gdn_decode/solution/triton/kernel.py:128-131); padding tokens: alpha = 1,
    // beta = 0. Cumulative decay in log2 units: every factor below is 2^(non-positive
    // difference), one v_exp_f32 (results below 2^-126 flush to 0, i.e. underflow).
    // L is summed in fp64 and kept as a float pair hi + lo: with strong decays |L| reaches
    // 10^4..10^5 in a chunk, where one ulp of a single float is already a 0.3% error in a
    // factor 2^(L_t - L_j) of two tokens close to each other. The lo parts never enter the
    // 64x64 matrices: 2^(L_t - L_j) = 2^lo_t 2^(hi_t - hi_j) 2^-lo_j is a diagonal
    // similarity, I + A = D (I + A~) D^-1 with D = diag(2^lo) and A~ built from hi alone,
    // so T = D T~ D^-1 and U = D U~ with U~ = T~ diag(beta 2^-lo) R. Hence the record holds
    //   T'~ = T~ diag(beta_j 2^-lo_j),  P'~[t, j] = scale 2^lo_t 2^(hi_t - hi_j) q_t . k_j,
    //   dec~_j = 2^(L_C - L_j) 2^lo_j = 2^((hi_C - hi_j) + lo_C),
    // and the scan's O = scale gamma (Q S0^T) + P'~ U~ and S_C = gamma_C S0 + (dec~ U~)^T K
    // are unchanged. hi_t - hi_j is exact (Sterbenz) wherever the factor is not negligible.
    // The raw bf16 bits are kept until gates() converts them at the end of the unit: a
    // conversion here would make the gate wave wait for these loads at the unit's start.
    auto gate_in = [&](const Unit &U, uint32_t &a_in, uint32_t &b_in) {
        const int tl = U.tok0 + min(l, U.len - 1);
        a_in = p.a[(int64_t)tl * p.a_st + (int64_t)U.h * p.a_sh];
        b_in = p.b[(int64_t)tl * p.b_st + (int64_t)U.h * p.b_sh];
    };
    auto gates = [&](const Unit &U, uint32_t a_raw, uint32_t b_raw, int buf) {
        const float a_in = bf16_to_f32(a_raw), b_in = bf16_to_f32(b_raw);
        // log2 alpha = -exp(A_log) log2(1 + e^x) (x > 20: -exp(A_log) x log2 e), with the
        // hardware base-2 exp / log; beta = 1 / (1 + e^-b)
        constexpr float kLog2e = 1.44269504088896340736f;
        float L = 0.f, bt = 0.f;
        if (l < U.len) {
            const float x = a_in + p.dt_bias[(int64_t)U.h * p.dt_s];
            const float sp2 = x > 20.f ? x * kLog2e
                                       : __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(x * kLog2e));
            L = -expf(p.A_log[(int64_t)U.h * p.A_log_s]) * sp2;
            bt = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-b_in * kLog2e));
        }
        float Ll;
        wave_prefix_sum_pair(L, L, Ll);  // cumulative log2 decay
        const float Lend = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(L), 63)),
                    Lendl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(Ll), 63));
        sm.L[buf][hv][l] = L;
        sm.Llo[buf][hv][l] = Ll;
        sm.B[buf][hv][l] = bt;
        char *rec = p.records + ((int64_t)U.c * p.HV + U.h) * kRecBytes;
        float *gts = (float *)(rec + kRecGates);
        // 2^hi alone: its error is 2^-24 |L| relative, only above 2^-24 once 2^L < 2^-126
        const float gam = __builtin_amdgcn_exp2f(L);
        gts[l] = gam;
        gts[64 + l] = __builtin_amdgcn_exp2f((Lend - L) + Lendl);
        gts[128 + l] = p.scale * gam;
        if (l == 0)
            gts[192] = __builtin_amdgcn_exp2f(Lend);
        if (l < 4)
            ((float *)(rec + kRecZero))[l] = 0.f;
    };

    // MFMA operand: 16 rows, k-chunk 4 ks + lg.
    auto kop = [&](const u32x4 *M, int row, int ks) {
        return M[16 * row + ((4 * ks + lg) ^ pswz(row & 15))];
    };
    // Per-wave 16 x 16 fp32 tile: element (r, c) at column c ^ 4 (r / 4). Rows in pi order
    // (substitution, X_w) and in token order (transposes, T' staging) then read and write
    // without bank conflicts; 4-column groups stay contiguous for the f32x4 row reads.
    // (rows pi(lr) have r / 4 = lr % 4)
    float (*Ms)[16] = sm.Ms[wv];
    auto ms = [&](int r, int c, int rq) -> float & { return Ms[r][c ^ (rq << 2)]; };
    auto ms_row4 = [&](int r, int q, int rq) -> const f32x4 & {
        return *(const f32x4 *)&Ms[r][4 * (q ^ rq)];
    };

    // Diagonal-block masks of this lane, one bit per element: bits 0..3 keep P'[t][j] for
    // j <= t (t = 16 w + lr, j = 16 w + 4 lg + e), bits 4..7 keep A[t][j] for j < t
    // (t = 16 w + pi(lr), j = 16 w + 4 e + lg). They do not depend on w.
    int dbits0 = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        dbits0 |= (4 * lg + e <= lr) << e;
        dbits0 |= (4 * e + lg < pi16(lr)) << (4 + e);
    }
    auto compute = [&](const Unit &U, const u32x4 *Kb, int buf, uint32_t &na, uint32_t &nb,
                       const Unit &N, bool more) {
        char *rec = p.records + ((int64_t)U.c * p.HV + U.h) * kRecBytes;
        const float *Ls = sm.L[buf][hv], *Bs = sm.B[buf][hv];
        // token 16 w + lr: its row of P'~ and its column of T'~ carry 2^+-lo
        const float lo_w = sm.Llo[buf][hv][16 * w + lr];
        // re-derived per unit, so the compiler keeps one register instead of hoisting a
        // lane mask per element out of the unit loop (they spilled to VGPR lanes)
        int dbits = dbits0;
        asm volatile("" : "+v"(dbits));

        // P' row block w: lane (t = 16 w + lr, lg) holds columns 16 jb + 4 lg .. +3. All
        // blocks' MFMAs issue before any scaling / store, which then never waits on them.
        {
            const int t = 16 * w + lr;
            const float Lt = Ls[t], sct = p.scale * __builtin_amdgcn_exp2f(lo_w);
            u32x4 qn[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                qn[ks] = kop(sm.Q, t, ks);
            f32x4 rp[4];
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
                if (jb > w)
                    break;
                rp[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    rp[jb] = mfma_bf16(kop(Kb, 16 * jb + lr, ks), qn[ks], rp[jb]);
            }
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
                if (jb > w)
                    break;
                const f32x4 Lj = *(const f32x4 *)&Ls[16 * jb + 4 * lg];
                float pv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    pv[e] = sct * __builtin_amdgcn_exp2f(Lt - Lj[e]) * rp[jb][e];
                if (jb == w) {  // diagonal block: zero above the diagonal
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        pv[e] = keep_if(pv[e], dbits, e);
                }
                *(u32x2 *)(rec + kRecP + 2 * (tri_blk(w, jb) * kBlk + lr * 16 + 4 * lg)) =
                    u32x2{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
            }
        }

        // A column block w: lane (lr, lg) element e = A[16 i + pi(lr)][16 w + 4 e + lg],
        // blocks i = w .. 3; MFMAs first, then scaling.
        f32x4 Aww = {0.f, 0.f, 0.f, 0.f};
        {
            u32x4 kw[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                kw[ks] = kop(Kb, 16 * w + pi16(lr), ks);
            f32x4 ra[4];
#pragma unroll
            for (int i = 3; i >= 0; --i) {
                if (i < w)
                    break;
                ra[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    ra[i] = mfma_bf16(kw[ks], kop(Kb, 16 * i + pi16(lr), ks), ra[i]);
            }
            float Lm[4];  // columns 16 w + 4 e + lg
#pragma unroll
            for (int e = 0; e < 4; ++e)
                Lm[e] = Ls[16 * w + 4 * e + lg];
#pragma unroll
            for (int i = 3; i >= 0; --i) {
                if (i < w)
                    break;
                const int t = 16 * i + pi16(lr);
                const float Lt = Ls[t], btt = Bs[t];
                f32x4 av;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    av[e] = btt * __builtin_amdgcn_exp2f(Lt - Lm[e]) * ra[i][e];
                if (i == w) {  // diagonal block: strictly lower part only
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        av[e] = keep_if(av[e], dbits, 4 + e);
                    Aww = av;
                } else
                    sm.AO[hv][i * (i - 1) / 2 + w][l] = split4(av);
            }
        }

        // X_w = (I + A_ww)^-1. Lane (lr, lg) holds row pi(lr), columns lg + 4 s (s = 0..3)
        // of X; step m subtracts A[r][m] x (row m of X), row m being final (A is strictly
        // lower, so rows r <= m see A[r][m] = 0). Row m sits in lane pi(m) of every 16-lane
        // row, next to the same columns.
        f32x4 xw;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            ms(pi16(lr), 4 * e + lg, lr & 3) = -Aww[e];
        {
            float arow[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 v = ms_row4(pi16(lr), q, lr & 3);
                arow[4 * q] = v[0]; arow[4 * q + 1] = v[1]; arow[4 * q + 2] = v[2]; arow[4 * q + 3] = v[3];
            }
            float x[4];
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2)
                x[s2] = pi16(lr) == lg + 4 * s2 ? 1.f : 0.f;
            // x enters the asm, so its initialisation is done before the nop: the first DPP
        // read of each x[s2] then has the two wait states a VALU write needs before it
        asm volatile("s_nop 1" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]) : : "memory");
            // arow holds -A; the broadcast lane of step M is pi(M)
#define GDN_SUBST_STEP(M, K)                                                      \
            GDN_FMAC_BCAST(x[0], arow[M], K); GDN_FMAC_BCAST(x[1], arow[M], K);   \
            GDN_FMAC_BCAST(x[2], arow[M], K); GDN_FMAC_BCAST(x[3], arow[M], K);
            GDN_SUBST_STEP(0, 0) GDN_SUBST_STEP(1, 4) GDN_SUBST_STEP(2, 8) GDN_SUBST_STEP(3, 12)
            GDN_SUBST_STEP(4, 1) GDN_SUBST_STEP(5, 5) GDN_SUBST_STEP(6, 9) GDN_SUBST_STEP(7, 13)
            GDN_SUBST_STEP(8, 2) GDN_SUBST_STEP(9, 6) GDN_SUBST_STEP(10, 10) GDN_SUBST_STEP(11, 14)
            GDN_SUBST_STEP(12, 3) GDN_SUBST_STEP(13, 7) GDN_SUBST_STEP(14, 11)
#undef GDN_SUBST_STEP
            xw = f32x4{x[0], x[1], x[2], x[3]};
        }
        sm.XA[hv][w][l] = split4(xw);
        // X_w in B-operand layout (lane (n, lg) element s = X[4 s + lg][n]) via the scratch
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
            ms(pi16(lr), lg + 4 * s2, lr & 3) = xw[s2];
        f32x4 TB[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
            TB[0][s2] = ms(4 * s2 + lg, lr, s2);
        // every X_i is in XA, every A_im in AO; every wave is done with Q (the next unit's K
        // copy stays in flight)
        lds_barrier_inflight();
        if (more)
            copy(N, true, sm.Q);

        // Column block w of T; TB[i] = T_(w+i),w in B-operand layout.
        // T_iw = -X_i z, z = sum_m A_im T_mw, with every 16x16x16 block product split into
        // bf16 hi / lo terms a_h b_h + a_l b_h + a_h b_l (a_l b_l, ~2^-16 relative, dropped).
        // An MFMA only pairs lane (m, g)'s k-slot j of A with lane (n, g)'s k-slot j of B, so
        // the fp32 operand layouts carry over (slot j = column 4 j + g), and a 16x16x32 MFMA
        // with A = [a_h | a_l], B = [b_h | b_h] computes two terms: column 0 takes 16 bf16
        // MFMAs instead of 36 fp32 ones at twice their cost.
        u32x4 TS[4];
        TS[0] = split4(TB[0]);
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            if (i + w > 3)
                break;
            u32x4 as[3];
#pragma unroll
            for (int m = 0; m < i; ++m) {  // A block (i + w, m + w)
                const int ii = i + w, mm = m + w;
                as[m] = sm.AO[hv][ii * (ii - 1) / 2 + mm][l];
            }
            f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < i; ++m)
                z = mfma_bf16(as[m], u32x4{TS[m][0], TS[m][1], TS[m][0], TS[m][1]}, z);
#pragma unroll
            for (int m = 0; m < i; m += 2) {
                if (m + 1 < i)
                    z = mfma_bf16(u32x4{as[m][0], as[m][1], as[m + 1][0], as[m + 1][1]},
                                  u32x4{TS[m][2], TS[m][3], TS[m + 1][2], TS[m + 1][3]}, z);
                else
                    z = mfma_bf16_k16(u32x2{as[m][0], as[m][1]}, u32x2{TS[m][2], TS[m][3]}, z);
            }
            const u32x4 xs = sm.XA[hv][i + w][l];
            const u32x4 zs = split4(z);
            f32x4 t = mfma_bf16(xs, u32x4{zs[0], zs[1], zs[0], zs[1]}, f32x4{0.f, 0.f, 0.f, 0.f});
            t = mfma_bf16_k16(u32x2{xs[0], xs[1]}, u32x2{zs[2], zs[3]}, t);
            TB[i] = -t;
            if (i + w < 3)
                TS[i] = split4(TB[i]);
        }

        // T'~ = T~ diag(beta 2^-lo) -> record (bf16 hi / lo, block layout), one block at a time
        // through this wave's fp32 staging tile: lane (row l / 4, columns 4 (l % 4) .. +3)
        // splits its four values and stores 8 bytes of hi and 8 of lo.
        const float bcol = Bs[16 * w + lr] * __builtin_amdgcn_exp2f(-lo_w);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i + w > 3)
                break;
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2)
                ms(4 * s2 + lg, lr, s2) = TB[i][s2] * bcol;
            const f32x4 v = ms_row4(l >> 2, l & 3, lg);
            uint32_t h01, l01, h23, l23;
            split_bf16x2(v[0], v[1], h01, l01);
            split_bf16x2(v[2], v[3], h23, l23);
            const int off = tri_blk(i + w, w) * 512 + (l >> 2) * 32 + 8 * (l & 3);
            *(u32x2 *)(rec + kRecThi + off) = u32x2{h01, h23};
            *(u32x2 *)(rec + kRecTlo + off) = u32x2{l01, l23};
        }

        // next unit's gates (its inputs were loaded one unit ago)
        if (more && w == kGateWave)
            gates(N, na, nb, buf ^ 1);
    };

    int u = blockIdx.x;
    if (u >= nunits)
        return;
    Unit U = unit(u);
    uint32_t a_in = 0, b_in = 0;
    copy(U, false, sm.K[0]);
    copy(U, true, sm.Q);
    if (w == kGateWave) {
        gate_in(U, a_in, b_in);
        gates(U, a_in, b_in, 0);
    }
    for (;;) {
        // even step: K in sm.K[0], gates in buffer 0
        int un = u + gridDim.x;
        bool more = un < nunits;
        Unit N = more ? unit(un) : U;
        dma_barrier();
        if (more) {
            copy(N, false, sm.K[1]);
            if (w == kGateWave)
                gate_in(N, a_in, b_in);
        }
        compute(U, sm.K[0], 0, a_in, b_in, N, more);
        if (!more)
            break;
        u = un;
        U = N;
        // odd step: K in sm.K[1], gates in buffer 1
        un = u + gridDim.x;
        more = un < nunits;
        N = more ? unit(un) : U;
        dma_barrier();
        if (more) {
            copy(N, false, sm.K[0]);
            if (w == kGateWave)
                gate_in(N, a_in, b_in);
        }
        compute(U, sm.K[1], 1, a_in, b_in, N, more);
        if (!more)
            break;
        u = un;
        U = N;
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
gdn_prefill_prep1_kernel(PrepArgs p)
{
    __shared__ PrepSmem<1> sm;
    prep_body<1>(p, sm);
}

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void
gdn_prefill_prep2_kernel(PrepArgs p)
{
    __shared__ PrepSmem<2> sm;
    prep_body<2>(p, sm);
}

}  // namespace gdn
