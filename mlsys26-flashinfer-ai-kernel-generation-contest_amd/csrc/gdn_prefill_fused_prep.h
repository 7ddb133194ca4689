// Prep of one chunk inside the fused prefill kernel: four prep waves build the chunk's
// T' = (I + A)^-1 diag(beta), P' and gate area for one v-head directly in the scan's LDS
// chunk buffer (the layouts the scan waves read: tlay, play, the gate area), from the
// chunk's K and Q, which the prep waves copy into that buffer themselves. The arithmetic
// is that of gdn_prefill_prep.hip (same gates, cumulative decay pair, similarity form,
// substitution and split-bf16 T chain); what differs is where operands come from and
// go to, and that the four prep waves synchronise among themselves with an LDS counter
// while the scan waves keep working on the previous chunk.
#pragma once

#include "gdn_prefill.h"

namespace gdn {

// LDS scratch of the prep waves (14 KB; with the scan's two chunk buffers the workgroup
// uses the whole 160 KB).
struct FusedPrepScratch {
    u32x4 XA[4][64];      // X_w = (I + A_ww)^-1 in A-operand layout, by lane, split4
    u32x4 AO[6][64];      // off-diagonal A_im (m < i) as XA; index i(i-1)/2 + m
    float Ms[4][16][16];  // per prep wave: -A_ww rows, X_w, then T' staging
};

constexpr int kPrepWaves = 4;
constexpr int kPrepSpin = 1 << 22;  // bound of a prep-wave wait (s_sleep 1 each, ~0.1 s)

// The prep waves' meeting point: every prep wave adds one to the counter (from its lane 0),
// then waits until all of them have (target = 4 x meetings so far). Waves of one workgroup are resident
// together, and every prep wave reaches every meeting, so the wait ends; it is still
// bounded (the results would then be wrong, and no wave hangs).
__device__ __forceinline__ void prep_meet(int *ctr, int target)
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    if ((threadIdx.x & 63) == 0)  // one count per wave
        __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    for (int it = 0; it < kPrepSpin; ++it) {
        if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target)
            break;
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Value of v held by lane src (all 64 lanes active).
__device__ __forceinline__ float lane_val(float v, int src)
{
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}

// One chunk (first token tok, lenc <= 64 tokens) of v-head h, by prep wave w (column block
// w, 0..3), into chunk buffer B. K and Q of the chunk are already in B (scan layouts: K row
// t, k-chunk c at unit 16 t + (c ^ kswz(t)); Q at 16 t + (c ^ (t & 15))); rows past lenc
// read as zero (they meet beta = 0 or the causal mask only). `meet` is the prep waves'
// meeting number before this chunk's internal meeting; it is advanced.
__device__ __forceinline__ void fused_prep_chunk(const ScanArgs &p, ScanBuf<8> &B,
                                                 FusedPrepScratch &ps, int *ctr, int &meet,
                                                 const int w, const int h, const int64_t tok,
                                                 const int lenc)
{
    const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;

    // Gates (gdn_decode/solution/triton/kernel.py:128-131) of token l, every prep wave
    // for itself (lanes read other tokens' values with lane_val); padding tokens: alpha =
    // 1, beta = 0. Cumulative log2 decay as a float pair hi + lo summed in fp64 (see the
    // gate notes of gdn_prefill_prep.hip: T', P', dec carry the similarity diag(2^lo)).
    float Lh, Ll, bt = 0.f;
    {
        const int64_t tl = tok + min(l, lenc - 1);
        const float a_in = bf16_to_f32(p.a[tl * p.a_st + (int64_t)h * p.a_sh]);
        const float b_in = bf16_to_f32(p.b[tl * p.b_st + (int64_t)h * p.b_sh]);
        constexpr float kLog2e = 1.44269504088896340736f;
        float L = 0.f;
        if (l < lenc) {
            const float x = a_in + p.dt_bias[(int64_t)h * p.dt_s];
            const float sp2 = x > 20.f ? x * kLog2e
                                       : __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(x * kLog2e));
            L = -expf(p.A_log[(int64_t)h * p.A_log_s]) * sp2;
            bt = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-b_in * kLog2e));
        }
        wave_prefix_sum_pair(L, Lh, Ll);
    }
    if (w == kPrepWaves - 1) {  // the gate area: gamma, dec, scale gamma, gammaC
        const float Lend = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(Lh), 63)),
                    Lendl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(Ll), 63));
        float *gts = (float *)B.G;
        const float gam = __builtin_amdgcn_exp2f(Lh);
        gts[l] = gam;
        gts[64 + l] = __builtin_amdgcn_exp2f((Lend - Lh) + Lendl);
        gts[128 + l] = p.scale * gam;
        if (l == 0)
            gts[192] = __builtin_amdgcn_exp2f(Lend);
    }

    auto kop = [&](int row, int ks) { return B.K[16 * row + ((4 * ks + lg) ^ kswz(row))]; };
    auto qop = [&](int row, int ks) { return B.Q[16 * row + ((4 * ks + lg) ^ (row & 15))]; };
    float(*Ms)[16] = ps.Ms[w];
    char *Tb0 = (char *)B.T[0], *Tb1 = (char *)B.T[1], *Pb = (char *)B.P;

    // Diagonal-block masks (as in gdn_prefill_prep.hip): bits 0..3 keep P'[t][j] for j <= t,
    // bits 4..7 keep A[t][j] for j < t.
    int dbits = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        dbits |= (4 * lg + e <= lr) << e;
        dbits |= (4 * e + lg < pi16(lr)) << (4 + e);
    }
    // token 16 w + lr: its row of P'~ and its column of T'~ carry 2^+-lo
    const float lo_w = lane_val(Ll, 16 * w + lr);

    // P' row block w: lane (t = 16 w + lr, lg) holds columns 16 jb + 4 lg .. +3; stored as
    // 8 bytes of LDS unit play(t, 2 jb + lg / 2).
    {
        const int t = 16 * w + lr;
        const float Lt = lane_val(Lh, t), sct = p.scale * __builtin_amdgcn_exp2f(lo_w);
        u32x4 qn[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            qn[ks] = qop(t, ks);
        f32x4 rp[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            if (jb > w)
                break;
            rp[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                rp[jb] = mfma_bf16(kop(16 * jb + lr, ks), qn[ks], rp[jb]);
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            if (jb > w)
                break;
            float pv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                pv[e] = sct * __builtin_amdgcn_exp2f(Lt - lane_val(Lh, 16 * jb + 4 * lg + e)) * rp[jb][e];
            if (jb == w) {  // diagonal block: zero above the diagonal
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    pv[e] = keep_if(pv[e], dbits, e);
            }
            *(u32x2 *)(Pb + 16 * play(t, 2 * jb + (lg >> 1)) + 8 * (lg & 1)) =
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
            kw[ks] = kop(16 * w + pi16(lr), ks);
        f32x4 ra[4];
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            if (i < w)
                break;
            ra[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                ra[i] = mfma_bf16(kw[ks], kop(16 * i + pi16(lr), ks), ra[i]);
        }
        float Lm[4];  // columns 16 w + 4 e + lg
#pragma unroll
        for (int e = 0; e < 4; ++e)
            Lm[e] = lane_val(Lh, 16 * w + 4 * e + lg);
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            if (i < w)
                break;
            const int t = 16 * i + pi16(lr);
            const float Lt = lane_val(Lh, t), btt = lane_val(bt, t);
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
                ps.AO[i * (i - 1) / 2 + w][l] = split4(av);
        }
    }

    // X_w = (I + A_ww)^-1 by forward substitution (gdn_prefill_prep.hip): lane (lr, lg)
    // holds row pi(lr), columns lg + 4 s of X; row m sits in lane pi(m) of every 16-lane row.
    f32x4 xw;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        Ms[pi16(lr)][4 * e + lg] = -Aww[e];
    {
        float arow[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 v = *(const f32x4 *)&Ms[pi16(lr)][4 * q];
            arow[4 * q] = v[0]; arow[4 * q + 1] = v[1]; arow[4 * q + 2] = v[2]; arow[4 * q + 3] = v[3];
        }
        float x[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
            x[s2] = pi16(lr) == lg + 4 * s2 ? 1.f : 0.f;
        // x enters the asm, so its initialisation is done before the nop: the first DPP
        // read of each x[s2] then has the two wait states a VALU write needs before it
        asm volatile("s_nop 1" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]) : : "memory");
#define GDN_SUBST_STEP(M, K)                                                      \
        GDN_FMAC_BCAST(x[0], arow[M], K); GDN_FMAC_BCAST(x[1], arow[M], K);       \
        GDN_FMAC_BCAST(x[2], arow[M], K); GDN_FMAC_BCAST(x[3], arow[M], K);
        GDN_SUBST_STEP(0, 0) GDN_SUBST_STEP(1, 4) GDN_SUBST_STEP(2, 8) GDN_SUBST_STEP(3, 12)
        GDN_SUBST_STEP(4, 1) GDN_SUBST_STEP(5, 5) GDN_SUBST_STEP(6, 9) GDN_SUBST_STEP(7, 13)
        GDN_SUBST_STEP(8, 2) GDN_SUBST_STEP(9, 6) GDN_SUBST_STEP(10, 10) GDN_SUBST_STEP(11, 14)
        GDN_SUBST_STEP(12, 3) GDN_SUBST_STEP(13, 7) GDN_SUBST_STEP(14, 11)
#undef GDN_SUBST_STEP
        xw = f32x4{x[0], x[1], x[2], x[3]};
    }
    ps.XA[w][l] = split4(xw);
    // X_w in B-operand layout (lane (n, lg) element s = X[4 s + lg][n]) via the staging tile
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
        Ms[pi16(lr)][lg + 4 * s2] = xw[s2];
    f32x4 TB[4];
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
        TB[0][s2] = Ms[4 * s2 + lg][lr];
    // every X_i is in XA, every A_im in AO
    meet += kPrepWaves;
    prep_meet(ctr, meet);

    // Column block w of T (split-bf16 chain, gdn_prefill_prep.hip): TB[i] = T_(w+i),w.
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
            as[m] = ps.AO[ii * (ii - 1) / 2 + mm][l];
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
        const u32x4 xs = ps.XA[i + w][l];
        const u32x4 zs = split4(z);
        f32x4 t = mfma_bf16(xs, u32x4{zs[0], zs[1], zs[0], zs[1]}, f32x4{0.f, 0.f, 0.f, 0.f});
        t = mfma_bf16_k16(u32x2{xs[0], xs[1]}, u32x2{zs[2], zs[3]}, t);
        TB[i] = -t;
        if (i + w < 3)
            TS[i] = split4(TB[i]);
    }

    // T'~ = T~ diag(beta 2^-lo): through the staging tile, lane (row l / 4, columns 4 (l % 4)
    // .. +3 of block (i + w, w)) splits four values into 8 bytes of hi and 8 of lo, stored
    // in LDS unit tlay(row, 2 w + (l % 4) / 2) of T' hi and lo.
    const float bcol = lane_val(bt, 16 * w + lr) * __builtin_amdgcn_exp2f(-lo_w);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (i + w > 3)
            break;
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
            Ms[4 * s2 + lg][lr] = TB[i][s2] * bcol;
        const f32x4 v = *(const f32x4 *)&Ms[l >> 2][4 * (l & 3)];
        uint32_t h01, l01, h23, l23;
        split_bf16x2(v[0], v[1], h01, l01);
        split_bf16x2(v[2], v[3], h23, l23);
        const int off = 16 * tlay(16 * (i + w) + (l >> 2), 2 * w + ((l & 3) >> 1)) + 8 * (l & 1);
        *(u32x2 *)(Tb0 + off) = u32x2{h01, h23};
        *(u32x2 *)(Tb1 + off) = u32x2{l01, l23};
    }
}

}  // namespace gdn
