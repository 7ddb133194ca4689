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
// Launches on the caller's stream:
//   plan  (1 + Z workgroups): sequence -> chunk tables from cu_seqlens on the device
//         (no host sync), longest-first sequence order, and zero-fill of output rows
//         that belong to no sequence. Skipped for 1 to 64 sequences, where the prep
//         kernel does the same work itself (PrepArgs::self_plan).
//   prep  (chunks x q/k heads): K K^T and Q K^T on MFMA, gates, cumulative log
//         decay, T = (I + A)^-1 (16x16 diagonal blocks by fp32 substitution,
//         off-diagonal blocks on split-bf16 MFMA), P; writes per (chunk, v-head) records.
//   scan  (sequences x v-heads): one workgroup owns 16 NW state rows of one
//         (sequence, v-head) and walks its chunks in order, state in registers.
//         fp32-valued operands on the state path (S0, R, T, U) are split into bf16
//         hi + lo halves so the state keeps ~2^-16 relative accuracy. With few
//         sequences, long ones are cut into segments scanned in parallel (two scan
//         launches over job tables).
//
// Files: gdn_prefill.h (records, layouts, argument structs, shared helpers),
// gdn_prefill_plan.hip, gdn_prefill_prep.hip, gdn_prefill_scan.hip (the kernels) and
// gdn_prefill.hip (workspace layout and launches behind gdn_prefill_launch).
#pragma once

#include "gdn_common.h"

namespace gdn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// A lone 4-slot term as a 16x16x32 MFMA with zero upper halves (a 16x16x16 MFMA costs the
// same ~16.7 cycles on gfx950)
__device__ __forceinline__ f32x4 mfma_bf16_k16(u32x2 a, u32x2 b, f32x4 c)
{
    return mfma_bf16(u32x4{a[0], a[1], 0u, 0u}, u32x4{b[0], b[1], 0u, 0u}, c);
}

// v if bit b of the lane's mask is set, else +0 (sign-extended bit field as an AND mask)
__device__ __forceinline__ float keep_if(float v, int bits, int b)
{
    return __int_as_float(__float_as_int(v) & __builtin_amdgcn_sbfe(bits, b, 1));
}

// Four floats split into bf16 hi / lo: {hi(v0, v1), hi(v2, v3), lo(v0, v1), lo(v2, v3)}, so
// .xy is a 4-element hi operand and the whole vector an 8-element [hi | lo] operand.
__device__ __forceinline__ u32x4 split4(f32x4 v)
{
    uint32_t h01, l01, h23, l23;
    split_bf16x2(v[0], v[1], h01, l01);
    split_bf16x2(v[2], v[3], h23, l23);
    return u32x4{h01, h23, l01, l23};
}

constexpr int kC = 64;   // chunk length
constexpr int kDK = 128; // head size

// Per (chunk, v-head) record in the workspace. 64x64 lower-triangular matrices are
// stored as their 10 lower 16x16 blocks, block (i, j <= i) at index i(i+1)/2 + j,
// each block row-major: exactly the rows and 8-column runs an MFMA A operand reads.
constexpr int kBlk = 256;        // elements per 16x16 block
// Byte offsets:
constexpr int kRecThi = 0;       // bf16 [10][16][16]  T' = (I + A)^-1 diag(beta), high half
constexpr int kRecTlo = 5120;    // bf16 [10][16][16]  low half
constexpr int kRecP = 10240;     // bf16 [10][16][16]  P' = scale * P (decayed, causal Q K^T)
constexpr int kRecGates = 15360; // f32 gamma[64], dec[64], scale * gamma[64], gammaC
// T', P' and dec are held up to a diagonal similarity diag(2^lo) that carries the low part
// of the cumulative log decay (gdn_prefill_prep.hip, gates); the scan uses them as they are.
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

// Barrier over LDS that leaves buffer_load ... lds copies in flight. Those copies write LDS
// and count in vmcnt, so the LDS release fence of lds_barrier waits for every one of them
// (vmcnt(0)); where the copies in flight target a buffer nobody reads before a later
// dma_barrier, waiting for this wave's own LDS operations (lgkmcnt(0)) is enough. The
// empty asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier_inflight()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt not waited for
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// DPP move with a row / bank mask: disabled rows and out-of-row sources read 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_or0(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWS, 0xF, true));
}

// dpp_or0 on 64-bit values (two 32-bit DPP moves)
template <int CTRL, int ROWS>
__device__ __forceinline__ int64_t dpp_or0_b64(int64_t v)
{
    const int lo = __builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, true),
              hi = __builtin_amdgcn_update_dpp(0, (int)(v >> 32), CTRL, ROWS, 0xF, true);
    return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_or0_f64(double x)
{
    return __longlong_as_double(dpp_or0_b64<CTRL, ROWS>(__double_as_longlong(x)));
}

// Inclusive prefix sum of int64 over the 64 lanes (the lane pattern of
// wave_prefix_sum_pair below).
__device__ __forceinline__ int64_t wave_prefix_sum_i64(int64_t x)
{
    x += dpp_or0_b64<0x111, 0xF>(x);
    x += dpp_or0_b64<0x112, 0xF>(x);
    x += dpp_or0_b64<0x114, 0xF>(x);
    x += dpp_or0_b64<0x118, 0xF>(x);
    x += dpp_or0_b64<0x142, 0xA>(x);
    x += dpp_or0_b64<0x143, 0xC>(x);
    return x;
}

// Inclusive prefix sum over the 64 lanes: shifts by 1, 2, 4, 8 inside each 16-lane row,
// then row 0's total into row 1 and row 2's into row 3 (row_bcast:15), then the total of
// rows 0-1 into rows 2-3 (row_bcast:31). Carried in fp64 (v_add_f64 is full rate) and
// returned as an unevaluated pair hi + lo of floats, hi the correctly rounded sum: lanes
// combine different partial sums, so single-float prefix sums of large values differ by an
// ulp where the exact sums are equal, while the pair keeps every difference of two lanes'
// sums to ~2^-48 of their size.
__device__ __forceinline__ void wave_prefix_sum_pair(float x, float &hi, float &lo)
{
    double s = x;
    s += dpp_or0_f64<0x111, 0xF>(s);
    s += dpp_or0_f64<0x112, 0xF>(s);
    s += dpp_or0_f64<0x114, 0xF>(s);
    s += dpp_or0_f64<0x118, 0xF>(s);
    s += dpp_or0_f64<0x142, 0xA>(s);
    s += dpp_or0_f64<0x143, 0xC>(s);
    hi = (float)s;
    lo = (float)(s - (double)hi);
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

// Segment jobs. When (sequence, v-head) pairs are too few to fill the GPU, a long sequence
// is cut into G segments scanned in parallel. The state map of a segment is affine,
// S_out = S_in M_s + R_s. Pass A scans segment 0 from the true initial state, giving
// S_in(1), and every middle segment s = 1 .. G - 2 twice from known states: value rows from
// zero give R_s, identity rows with V = 0 give M_s. Pass C rescans each segment s >= 1 for
// its outputs; its workgroups first chain S_in(s) = S_in(1) M_1 + R_1 ... (s - 1 steps) on
// their own state rows, and the last segment's scan ends in the final state, so the last
// segment needs no state map.
constexpr int kJobFirst = 0;   // from the initial state; outputs; final state -> new_state,
                               // or (slot >= 0) -> S_in(1)
constexpr int kJobZero = 1;    // value rows from a zero state, no outputs: final state = R_s
constexpr int kJobIdent = 2;   // identity rows with V = 0, no outputs: final state = M_s,
                               // stored as bf16 hi / lo units of M^T
constexpr int kJobResume = 3;  // from S_in(1) and (steps) chain steps; outputs; final state
                               // -> new_state for the last segment
// Slots hold one 128 x 128 fp32 matrix per (slot, v-head), each in the order its reader
// wants, so that every copy reads whole lines:
// * S_in(1) and R_s: register image of the scan's state layout, 16-byte unit
//   (8 (row / 16) + t) 64 + lane holds row 16 (row / 16) + lane % 16, columns
//   32 (t / 2) + 8 (lane / 16) + 4 (t % 2) + 0..3;
// * M_s: LDS image of M_s^T split into bf16 hi units (0 .. 2047) then lo units; unit
//   16 j + (cu ^ kswz(j)) holds M_s[8 cu .. 8 cu + 7][j].
constexpr int64_t kSlotFloats = 128 * 128;
// Job entry: {sequence, kind, first chunk, end chunk, slot, chain steps, last, the sequence's
// first token, length and first chunk, 0 ...}: a scan workgroup reads what it needs in one
// round of loads, issued together with the job count's.
constexpr int kJobInts = 16;
constexpr int kMtUnits = 2048;
constexpr int kSegMinChunks = 4;            // shortest segment (before balancing)
constexpr int kSegMaxG = 16;                // segments per sequence at most
// Segment lengths balance the two passes (measured on MI355X): a segment-0 chunk, which
// writes outputs in pass A, costs ~1/0.83 of a state-map chunk, and each chain step
// delays a pass-C segment by ~0.9 chunk-times, so segment s >= 1 gets 0.9 (s - 1) chunks
// fewer than segment 1.
constexpr float kSegFirstWeight = 0.83f;
constexpr float kSegChainChunks = 0.9f;

// ------------------------------------------------------------------------- plan
struct PlanArgs {
    const void *cu;
    int cu64, N, T, HO, nc;  // nc: chunk-table capacity (workspace bound)
    int32_t *header, *chunk_tok0, *chunk_len, *seq_chunk0, *seq_tok0, *seq_len;
    // longest-first order: seq_rank[4 r .. 4 r + 3] = {sequence, first token, length, first
    // chunk} of the r-th longest sequence (one 16-byte load per scan workgroup)
    int32_t *seq_rank;
    bf16_t *out;
    int64_t o_st, o_sh;
    // segments (seg_G >= 3): at most seg_G segments per sequence; job entries of kJobInts
    // ints, pass A from jobs[0], pass C from jobs[kJobInts seg_capA]; counts in header[1]
    // (pass A) and header[2] (pass C). seg_c4 > 0: pass C is launched twice, with 4 and with
    // 8 waves per workgroup; a plan with at most seg_c4 pass-C jobs (128 (job, v-head) pairs)
    // counts them in header[2] for the 4-wave launch, a larger one in header[3] for the
    // 8-wave launch, and the other launch finds no job.
    int seg_G, seg_capA, seg_c4;
    // whole_cus > 0 (whole sequences, the 4-wave and the 8-wave scan both launched, this many
    // CUs): the planner gives the sequences to the 4-wave launch (header[4] = N, header[5] = 0)
    // when it is the faster, else to the 8-wave launch (header[4] = 0, header[5] = N)
    int whole_cus;
    int32_t *jobs;
};

constexpr int kPlanSortMax = 512;

// Maximum over the 64 lanes of non-negative values (the prefix pattern of
// wave_prefix_sum_i64; lane 63 holds the total), returned to every lane.
__device__ __forceinline__ float wave_max_nonneg(float x)
{
    x = fmaxf(x, dpp_or0<0x111, 0xF>(x));
    x = fmaxf(x, dpp_or0<0x112, 0xF>(x));
    x = fmaxf(x, dpp_or0<0x114, 0xF>(x));
    x = fmaxf(x, dpp_or0<0x118, 0xF>(x));
    x = fmaxf(x, dpp_or0<0x142, 0xA>(x));
    x = fmaxf(x, dpp_or0<0x143, 0xC>(x));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// Segment job tables, built by one wave with all 64 lanes active (at most 64 sequences:
// the host asks for segments only then), lane i for the sequence of rank i (order[i],
// longest first), from each sequence's first chunk (clamped to nc) and token count.
//
// Estimates count in pass-C chunk times: a pass-A chunk with outputs weighs
// 1 / kSegFirstWeight, a state-map chunk 1, a chain step kSegChainChunks. A sequence of
// at least 3 kSegMinChunks chunks is cut into G balanced segments (segment 0 weighted by
// kSegFirstWeight, each later one kSegChainChunks chunks shorter than the one before, so
// that both passes take `base` chunk times); G is the largest balanced count, at most
// seg_G and len / kSegMinChunks, below the minimum of 2 base(G) over real G,
// G* = 1 - w + sqrt(w^2 + w + len / h) with w = kSegFirstWeight, h = kSegChainChunks / 2.
// Shorter sequences stay whole and run in whichever pass they lengthen least; a whole
// job is a kJobFirst entry without a slot, which either pass runs. When the longest
// sequence scanned whole is no longer than the two spans plus one chunk time (a second
// pass's start), nothing is cut and every sequence runs whole in pass C.
// Pass A lists every segment 0 and whole sequence first (rank order), then the state maps;
// slots q .. q + G - 2 of a cut sequence hold S_in(1) and M_s, R_s of the middle segments
// s (slot q + s - 1).
__device__ inline void plan_jobs(const PlanArgs &p, const int32_t *order, const int32_t *first,
                                 const int32_t *tok0, const int32_t *len, int lane)
{
    constexpr float w = kSegFirstWeight, h = 0.5f * kSegChainChunks;
    const bool act = lane < p.N;
    const int n = act ? order[lane] : 0;
    int ncks = 0;
    if (act) {
        const int f = first[n], e = min(f + (len[n] + kC - 1) / kC, p.nc);
        ncks = e - f;
    }
    auto base_of = [&](int g) { return (ncks + h * (g - 1) * (g - 2)) / (w + g - 1); };
    auto balanced = [&](int g, float b) {
        return b - kSegChainChunks * (g - 2) >= 2.f && w * b >= 2.f;
    };
    int G = 1;
    float base = 0.f;
    const int gmax = min(p.seg_G, ncks / kSegMinChunks);
    if (gmax >= 3) {
        const float gs = 1.f - w + sqrtf(w * w + w + ncks / h);
        int g = max(3, min(gmax, (int)gs));
        float b = base_of(g);
        while (g > 3 && !balanced(g, b))
            b = base_of(--g);
        G = g;
        base = b;
    }
    const bool bal = G > 1 && balanced(G, base);
    const int Ls = G > 1 ? (ncks + G - 1) / G : ncks;
    if (G > 1 && !bal) {  // equal lengths: as many segments as Ls-chunk pieces
        G = (ncks + Ls - 1) / Ls;
        if (G < 3)
            G = 1;
    }
    // first chunk of segment sg
    auto bnd = [&](int sg) {
        if (sg >= G)
            return ncks;
        if (!bal)
            return min(sg * Ls, ncks);
        const float x = w * base + (sg - 1) * base - h * (sg - 1) * (sg - 2);
        return min(max((int)(x + 0.5f), sg), ncks);
    };
    // pass spans of the cut sequences
    float sa = 0.f, sc = 0.f;
    if (G > 1) {
        sa = bnd(1) / w;
        for (int sg = 1; sg < G; ++sg) {
            const int ls = bnd(sg + 1) - bnd(sg);
            if (sg < G - 1)
                sa = fmaxf(sa, (float)ls);
            sc = fmaxf(sc, ls + kSegChainChunks * (sg - 1));
        }
    }
    float spanA = wave_max_nonneg(sa), spanC = wave_max_nonneg(sc);
    const float cmax = wave_max_nonneg((float)ncks);
    // whole sequences, longest first: each to the pass it lengthens least (ties: A); once
    // one fits both spans, every shorter one does too
    uint64_t in_c = 0;
    for (int i = 0; i < p.N; ++i) {
        const int gi = __builtin_amdgcn_readlane(G, i);
        const float c = (float)__builtin_amdgcn_readlane(ncks, i);
        if (gi > 1)
            continue;
        if (c / w <= spanA && c <= spanC)
            break;
        if (fmaxf(spanA, c / w) - spanA <= fmaxf(spanC, c) - spanC) {
            spanA = fmaxf(spanA, c / w);
        } else {
            spanC = fmaxf(spanC, c);
            in_c |= uint64_t(1) << i;
        }
    }
    const bool whole_all = cmax <= spanA + spanC + 1.f;
    const bool whole = whole_all || G == 1;
    const bool wc = whole_all || ((in_c >> lane) & 1);
    // job counts -> offsets (exclusive prefix sums in rank order)
    const int firstA = act && !(whole && wc), mapsA = act && !whole ? 2 * (G - 2) : 0;
    const int passC = !act ? 0 : whole ? (wc ? 1 : 0) : G - 1;
    const int slots = act && !whole ? G - 1 : 0;
    const int64_t iF = wave_prefix_sum_i64(firstA), iM = wave_prefix_sum_i64(mapsA),
                  iC = wave_prefix_sum_i64(passC), iS = wave_prefix_sum_i64(slots);
    const int totF = (int)__builtin_amdgcn_readlane((int)iF, 63),
              totM = (int)__builtin_amdgcn_readlane((int)iM, 63),
              totC = (int)__builtin_amdgcn_readlane((int)iC, 63);
    int oF = (int)iF - firstA, oM = totF + (int)iM - mapsA, oC = p.seg_capA + (int)iC - passC;
    const int q = (int)iS - slots;
    const int t0n = act ? tok0[n] : 0, lenn = act ? len[n] : 0, c0n = act ? first[n] : 0;
    auto put = [&](int idx, int kind, int cb, int ce, int slot, int steps, int last) {
        int4 *e = (int4 *)(p.jobs + kJobInts * idx);
        e[0] = int4{n, kind, cb, ce};
        e[1] = int4{slot, steps, last, t0n};
        e[2] = int4{lenn, c0n, 0, 0};
    };
    if (act) {
        if (whole) {
            put(wc ? oC : oF, kJobFirst, 0, ncks, -1, 0, 0);
        } else {
            put(oF, kJobFirst, 0, bnd(1), q, 0, 0);
            for (int sg = 1; sg < G; ++sg) {
                const int cb = bnd(sg), ce = bnd(sg + 1);
                if (sg < G - 1) {
                    put(oM++, kJobZero, cb, ce, q + sg - 1, 0, 0);
                    put(oM++, kJobIdent, cb, ce, q + sg - 1, 0, 0);
                }
                put(oC++, kJobResume, cb, ce, q, sg - 1, sg == G - 1);
            }
        }
    }
    if (lane == 0) {
        const bool c8 = p.seg_c4 > 0 && totC > p.seg_c4;
        p.header[1] = totF + totM;
        p.header[2] = c8 ? 0 : totC;
        p.header[3] = c8 ? totC : 0;
    }
}

// ------------------------------------------------------------------------- LDS copies
#define GDN_LDS __attribute__((address_space(3)))
typedef short s16x4 __attribute__((ext_vector_type(4)));

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): lane i writes
// dst + 16 i; dst is wave-uniform, src is per lane.
__device__ __forceinline__ void dma16(const char *src, void *dst)
{
    __builtin_amdgcn_global_load_lds((const void *)src, (GDN_LDS void *)dst, 16, 0, 0);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane n receives element n % 4 of the
// four 8-byte pieces addressed by lanes n / 4 + 4 r, r = 0..3 (element r of the result).
__device__ __forceinline__ u32x2 lds_tr16(const void *p)
{
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GDN_LDS s16x4 *)p);
    return __builtin_bit_cast(u32x2, r);
}

// Wait for this wave's LDS copies, then for the whole workgroup.
__device__ __forceinline__ void dma_barrier()
{
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    lds_barrier();
}

// ------------------------------------------------------------------------- prep
struct PrepArgs {
    const bf16_t *q, *k, *a, *b;
    const float *A_log, *dt_bias;
    // element strides, host-checked to fit 31 bits (32-bit here keeps scalar registers free)
    int32_t q_st, q_sh, k_st, k_sh, a_st, a_sh, b_st, b_sh, A_log_s, dt_s;
    const int32_t *header, *chunk_tok0, *chunk_len;
    char *records;
    int HQK, HV, ratio;
    float scale;
    // Self-planned launch (1 <= N <= kSelfPlanMax; no plan kernel): every workgroup finds
    // its units' chunks from cu_seqlens itself, the last block writes the tables the scan reads
    // (plan.header, seq_*, jobs) and the workgroups zero-fill the output rows outside every
    // sequence. Otherwise the plan kernel ran first and header / chunk_* hold its tables.
    int self_plan;
    PlanArgs plan;
};

constexpr int kSelfPlanMax = 64;  // one sequence per lane of a wave

// ------------------------------------------------------------------------- scan
struct ScanArgs {
    const bf16_t *q, *k, *v;
    const float *state;
    float *new_state;
    bf16_t *out;
    int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh;
    int64_t st_sn, st_sh, st_sv, ns_sn, ns_sh, ns_sv;
    const int32_t *header, *seq_chunk0, *seq_tok0, *seq_len, *seq_rank;
    const char *records;
    int HQK, HV, ratio, ngroups;
    // Segment jobs (jobs != nullptr): the grid walks entries jobs[kJobInts (job_first + e)]
    // for e < header[njob_idx] instead of whole sequences. Whole sequences (jobs == nullptr)
    // with njob_idx > 0: only the sequences of rank < header[njob_idx] are scanned (the
    // planner hands all or none of them to this launch). Slot buffers hold one 128 x 128
    // fp32 matrix per (slot, v-head): S_in(1) (seg_sin), R_s (seg_r), or M_s as bf16 hi /
    // lo units (seg_mt, kMtUnits).
    const int32_t *jobs;
    int job_first, njob_idx;
    float *seg_sin, *seg_r, *seg_mt;
};


// LDS layouts (16-byte units). A ds_read_b128 is served in four cycles of 16 lanes: the
// lanes of one 32-lane half whose lane bits 2, 3, 4 have equal parity; a cycle is
// conflict-free when its 16 lanes touch 16 distinct units modulo 256 bytes (measured on
// gfx950). Every b128 operand read below meets that:
//   K row t, k-chunk c (k = 8c .. 8c+7)   -> unit 16 t + (c ^ kswz(t))
//   Q row t, k-chunk c                    -> unit 16 t + (c ^ (t & 15))
//   V row t, v-chunk c                    -> unit 2 NW t + (c ^ 2 (t & 3))
//   T' row r, column chunk c (8 columns)  -> unit tlay(r, c)
//   P' row r, column chunk c              -> unit play(r, c)
// T' is read with rows in the permuted order of the X / U tiles, P' in token order; both
// layouts are bit permutations of (r, c) that put a read's four free lane bits into the
// low unit bits and its tile / k-step into high ones (additive offsets).
__host__ __device__ constexpr int kswz(int t)
{
    return ((t & 1) ? 1 : 0) ^ ((t & 2) ? 14 : 0) ^ ((t & 8) ? 6 : 0) ^ ((t & 16) ? 4 : 0);
}
__host__ __device__ constexpr int tlay(int r, int c)
{
    return (r & 3) | (((r >> 3) & 1) << 2) | ((c & 1) << 3) | (((r >> 4) & 1) << 4) |
           (((c >> 1) & 1) << 5) | ((c >> 2) << 6) | (((r >> 2) & 1) << 7) | ((r >> 5) << 8);
}
__host__ __device__ constexpr int play(int r, int c)
{
    return (r & 7) | ((c & 1) << 3) | (((r >> 3) & 1) << 4) | (((c >> 1) & 1) << 5) |
           ((c >> 2) << 6) | (((r >> 4) & 1) << 7) | ((r >> 5) << 8);
}
// Inverses (unit -> row, column chunk), used by the record copies.
__host__ __device__ constexpr int tlay_row(int u)
{
    return (u & 3) | (((u >> 7) & 1) << 2) | (((u >> 2) & 1) << 3) | (((u >> 4) & 1) << 4) |
           ((u >> 8) << 5);
}
__host__ __device__ constexpr int play_row(int u)
{
    return (u & 7) | (((u >> 4) & 1) << 3) | (((u >> 7) & 1) << 4) | ((u >> 8) << 5);
}
__host__ __device__ constexpr int lay_col(int u)
{
    return ((u >> 3) & 1) | (((u >> 5) & 1) << 1) | (((u >> 6) & 1) << 2);
}
constexpr bool layouts_invert()
{
    for (int r = 0; r < 64; ++r)
        for (int c = 0; c < 8; ++c)
            if (tlay_row(tlay(r, c)) != r || lay_col(tlay(r, c)) != c ||
                play_row(play(r, c)) != r || lay_col(play(r, c)) != c)
                return false;
    return true;
}
static_assert(layouts_invert(), "T' / P' LDS layouts must be bijections");

// Row order inside a 16-row block used for fp32 MFMA operands: pi(m) = 4 (m % 4) + m / 4
// (a 4 x 4 transpose, its own inverse). With pi-ordered rows an MFMA result in C layout
// (lane (n, g) holds rows 4 g + i) already holds rows 4 i + g: exactly the operand
// layout of the next v_mfma_f32_16x16x4_f32 (k-slice i, lane (n, g) supplies k = 4 i + g).
__device__ __forceinline__ int pi16(int m) { return 4 * (m & 3) + (m >> 2); }

// acc += coef * (acc of lane K in this 16-lane row): one v_fmac_f32 with a DPP row_newbcast
// source. Callers keep >= 2 other VALU instructions between the last write of acc and
// this read (the DPP read-after-write hazard); the first use in a chain is preceded by
// s_nop 1.
#define GDN_FMAC_BCAST(acc, coef, K)                                                     \
    asm volatile("v_fmac_f32_dpp %0, %0, %1 row_newbcast:" #K " row_mask:0xf bank_mask:0xf" \
                 : "+v"(acc)                                                              \
                 : "v"(coef))

// One chunk in LDS, as the workgroup's waves read it.
template <int NW>
struct ScanBuf {
    u32x4 K[kC * 16];      // 16 KB
    u32x4 Q[kC * 16];      // 16 KB
    u32x4 V[kC * 2 * NW];  // the workgroup's 16 NW value columns
    u32x4 T[2][512];       // T' hi / lo (tlay)
    u32x4 P[512];          // P' (play)
    f32x4 G[64];           // the record's gate area (gamma, dec, scale gamma, gammaC)
};

// ------------------------------------------------------------------------- kernels
// Defined in gdn_prefill_plan.hip, gdn_prefill_prep.hip and gdn_prefill_scan.hip; the
// scan kernels are instantiated there for SEG = false (whole sequences) and true
// (segment jobs).
__global__ __launch_bounds__(256) void gdn_prefill_plan_kernel(PlanArgs p);
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
gdn_prefill_prep1_kernel(PrepArgs p);
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void
gdn_prefill_prep2_kernel(PrepArgs p);
template <bool SEG>
__global__ __launch_bounds__(512) void gdn_prefill_scan8_kernel(ScanArgs p);
template <bool SEG>
__global__ __launch_bounds__(256) void gdn_prefill_scan4_kernel(ScanArgs p);

}  // namespace gdn
