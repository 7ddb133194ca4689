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

#include <algorithm>

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

// Inclusive prefix sum over the 64 lanes: shifts by 1, 2, 4, 8 inside each 16-lane row,
// then row 0's total into row 1 and row 2's into row 3 (row_bcast:15), then the total of
// rows 0-1 into rows 2-3 (row_bcast:31).
__device__ __forceinline__ float wave_prefix_sum(float x)
{
    x += dpp_or0<0x111, 0xF>(x);
    x += dpp_or0<0x112, 0xF>(x);
    x += dpp_or0<0x114, 0xF>(x);
    x += dpp_or0<0x118, 0xF>(x);
    x += dpp_or0<0x142, 0xA>(x);
    x += dpp_or0<0x143, 0xC>(x);
    return x;
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
constexpr int kMtUnits = 2048;
constexpr int kSegMinChunks = 4;            // shortest segment (before balancing)
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
    int32_t *header, *chunk_tok0, *chunk_len, *seq_chunk0, *seq_order, *seq_tok0, *seq_len;
    bf16_t *out;
    int64_t o_st, o_sh;
    // segments (seg_G >= 3): at most seg_G segments per sequence; job entries of 8 ints
    // {sequence, kind, first chunk, end chunk, slot, chain steps, last}, pass A from
    // jobs[0], pass C from jobs[8 seg_capA]; counts in header[1], header[2]
    int seg_G, seg_capA;
    int32_t *jobs;
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
        // up to kPlanSortMax sequences the chunk table is filled chunk-parallel from these
        __shared__ int32_t s_first[kPlanSortMax], s_end[kPlanSortMax], s_t0[kPlanSortMax],
            s_len[kPlanSortMax];
        __shared__ int64_t s_carry;
        const bool par = p.N <= kPlanSortMax;
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
                if (par) {
                    s_first[n] = (int32_t)(first < p.nc ? first : p.nc);
                    s_end[n] = (int32_t)(first + nck < p.nc ? first + nck : p.nc);
                    s_t0[n] = t0;
                    s_len[n] = ln;
                } else {
                    for (int i = 0; i < nck && first + i < p.nc; ++i) {
                        p.chunk_tok0[first + i] = t0 + i * kC;
                        p.chunk_len[first + i] = min(kC, ln - i * kC);
                    }
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
        if (par) {  // chunk c belongs to the first sequence whose chunks end after c
            __syncthreads();
            const int total = (int)(s_carry < p.nc ? s_carry : p.nc);
            for (int c = tid; c < total; c += 256) {
                int lo = 0, hi = p.N - 1;
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (s_end[mid] > c)
                        hi = mid;
                    else
                        lo = mid + 1;
                }
                const int i = c - s_first[lo];
                p.chunk_tok0[c] = s_t0[lo] + i * kC;
                p.chunk_len[c] = min(kC, s_len[lo] - i * kC);
            }
        }
        // Longest-first order (identity when N is large).
        __shared__ int32_t s_order[kPlanSortMax];
        if (p.N <= kPlanSortMax) {
            for (int n = tid; n < p.N; n += 256) {
                const int mine = s_nck[n];
                int rank = 0;
                for (int m = 0; m < p.N; ++m) {
                    const int o = s_nck[m];
                    rank += (o > mine) || (o == mine && m < n);
                }
                p.seq_order[rank] = n;
                s_order[rank] = n;
            }
        } else {
            for (int n = tid; n < p.N; n += 256)
                p.seq_order[n] = n;
        }
        if (p.seg_G >= 3 && par) {  // segment job tables (host only asks for small N)
            __syncthreads();
            if (tid == 0) {
                auto put = [&](int idx, int n, int kind, int cb, int ce, int q, int steps, int last) {
                    int32_t *e = p.jobs + 8 * idx;
                    e[0] = n;
                    e[1] = kind;
                    e[2] = cb;
                    e[3] = ce;
                    e[4] = q;
                    e[5] = steps;
                    e[6] = last;
                };
                // pass A: every segment 0 first (longest sequences first), then the state
                // maps; slots q .. q + G - 2 of a sequence hold S_in(1) and M_s, R_s of the
                // middle segments s (slot q + s - 1)
                int na = 0, nc3 = 0;
                for (int pass = 0; pass < 2; ++pass) {
                    int qs = 0;
                    for (int i = 0; i < p.N; ++i) {
                        const int n = s_order[i];
                        const int ncks = s_end[n] - s_first[n];
                        int G = min(p.seg_G, max(1, ncks / kSegMinChunks));
                        const int Ls = (ncks + G - 1) / G;
                        G = Ls > 0 ? (ncks + Ls - 1) / Ls : 1;
                        if (G < 3)
                            G = 1;  // two segments would run one after the other
                        // boundary of segment sg: balanced lengths (see kSegFirstWeight) when
                        // every segment keeps at least 2 chunks, else equal lengths
                        const float base = (ncks + kSegChainChunks * (G - 1) * (G - 2) / 2) /
                                           (kSegFirstWeight + G - 1);
                        const bool bal = G > 1 && base - kSegChainChunks * (G - 2) >= 2.f &&
                                         kSegFirstWeight * base >= 2.f;
                        auto bnd = [&](int sg) {
                            if (sg >= G)
                                return ncks;
                            if (!bal)
                                return min(sg * Ls, ncks);
                            // chunks before segment sg: kSegFirstWeight base + sum over
                            // u = 1 .. sg - 1 of (base - kSegChainChunks (u - 1))
                            const float x = kSegFirstWeight * base + (sg - 1) * base -
                                            kSegChainChunks * (sg - 1) * (sg - 2) / 2;
                            return min(max((int)(x + 0.5f), sg), ncks);
                        };
                        const int q = G > 1 ? qs : -1;
                        qs += G - 1;
                        if (pass == 0) {
                            put(na++, n, kJobFirst, 0, G > 1 ? bnd(1) : ncks, q, 0, 0);
                            continue;
                        }
                        for (int sg = 1; sg < G; ++sg) {
                            const int cb = bnd(sg), ce = bnd(sg + 1);
                            if (sg < G - 1) {
                                put(na++, n, kJobZero, cb, ce, q + sg - 1, 0, 0);
                                put(na++, n, kJobIdent, cb, ce, q + sg - 1, 0, 0);
                            }
                            put(p.seg_capA + nc3++, n, kJobResume, cb, ce, q, sg - 1, sg == G - 1);
                        }
                    }
                }
                p.header[1] = na;
                p.header[2] = nc3;
            }
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
};

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
// wave (hv, 3), which has the least work after the barrier, also computes the next unit's
// gates and cumulative log2 decay L.
// (gdn_prefill/solution/triton/kernel.py:60-79 form the same A, T and P.)
template <int VH>
struct PrepSmem {
    u32x4 K[2][kC * 16];  // row t, k-chunk c at unit 16 t + (c ^ (t & 15))
    u32x4 Q[kC * 16];
    float L[2][VH][64];   // L by token
    float LT[2][VH][64];  // L of token 16 b + 4 i + g at 16 b + 4 g + i
    float B[2][VH][64];   // beta by token
    u32x4 XA[VH][4][64];  // X_w in A-operand layout, by lane, split4
    u32x4 AO[VH][6][64];  // off-diagonal A_im (m < i) as XA; index i(i-1)/2 + m
    float Ms[4 * VH][16][16];  // per wave: -A_ww rows, X_w, then T' staging
};

constexpr int kGateWave = 3;  // column block with no work after the barrier

template <int VH>
__device__ __forceinline__ void prep_body(const PrepArgs &p, PrepSmem<VH> &sm)
{
    const int ngrp = p.ratio / VH;
    const int nunits = p.header[0] * p.HQK * ngrp;
    // wv is wave-uniform: branches on the column block are scalar branches
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63,
              lr = l & 15, lg = l >> 4;
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
        r.tok0 = p.chunk_tok0[r.c];
        r.len = p.chunk_len[r.c];
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
            dma16(base + (uint32_t)min(t, U.len - 1) * st2 + 16u * (cs ^ (t & 15)), &dst[64 * b]);
        }
    };
    // Gates (gdn_decode/solution/triton/kernel.py:128-131); padding tokens: alpha = 1,
    // beta = 0. Cumulative decay in log2 units: every factor below is 2^(non-positive
    // difference), one v_exp_f32 (results below 2^-126 flush to 0, i.e. underflow).
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
        L = wave_prefix_sum(L);  // cumulative log2 decay
        const float Lend = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(L), 63));
        sm.L[buf][hv][l] = L;
        sm.B[buf][hv][l] = bt;
        sm.LT[buf][hv][16 * (l >> 4) + 4 * (l & 3) + ((l >> 2) & 3)] = L;
        char *rec = p.records + ((int64_t)U.c * p.HV + U.h) * kRecBytes;
        float *gts = (float *)(rec + kRecGates);
        const float gam = __builtin_amdgcn_exp2f(L);
        gts[l] = gam;
        gts[64 + l] = __builtin_amdgcn_exp2f(Lend - L);
        gts[128 + l] = p.scale * gam;
        if (l == 0)
            gts[192] = __builtin_amdgcn_exp2f(Lend);
        if (l < 4)
            ((float *)(rec + kRecZero))[l] = 0.f;
    };

    // MFMA operand: 16 rows, k-chunk 4 ks + lg.
    auto kop = [&](const u32x4 *M, int row, int ks) {
        return M[16 * row + ((4 * ks + lg) ^ (row & 15))];
    };
    float (*Ms)[16] = sm.Ms[wv];

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
        const float *Ls = sm.L[buf][hv], *Bs = sm.B[buf][hv], *LsT = sm.LT[buf][hv];
        // re-derived per unit, so the compiler keeps one register instead of hoisting a
        // lane mask per element out of the unit loop (they spilled to VGPR lanes)
        int dbits = dbits0;
        asm volatile("" : "+v"(dbits));

        // P' row block w: lane (t = 16 w + lr, lg) holds columns 16 jb + 4 lg .. +3. All
        // blocks' MFMAs issue before any scaling / store, which then never waits on them.
        {
            const int t = 16 * w + lr;
            const float Lt = Ls[t];
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
                    pv[e] = p.scale * __builtin_amdgcn_exp2f(Lt - Lj[e]) * rp[jb][e];
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
            const f32x4 Lm = *(const f32x4 *)&LsT[16 * w + 4 * lg];
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
            asm volatile("s_nop 1" ::: "memory");
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
            Ms[pi16(lr)][lg + 4 * s2] = xw[s2];
        f32x4 TB[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
            TB[0][s2] = Ms[4 * s2 + lg][lr];
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

        // T' = T diag(beta) -> record (bf16 hi / lo, block layout), one block at a time
        // through this wave's fp32 staging tile: lane (row l / 4, columns 4 (l % 4) .. +3)
        // splits its four values and stores 8 bytes of hi and 8 of lo.
        const float bcol = Bs[16 * w + lr];
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
    // Segment jobs (jobs != nullptr): the grid walks entries jobs[8 (job_first + e)] =
    // {sequence, kind, first chunk, end chunk, slot, chain steps, last} for
    // e < header[njob_idx] instead of whole sequences. Slot buffers hold one 128 x 128
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

// Copy windows of one chunk, 64 units (1 KB) each: K rows 4b..4b+3 (16 windows), Q (16),
// V (NW == 8: 4 rows per window, NW == 4: 8 rows), then 6 windows each of T' hi, T' lo
// and P' and the gate area. Each record window fills LDS units 64 b .. 64 b + 63 of its
// matrix (b = 0, 2, 4, 5, 6, 7; windows 1 and 3 hold rows 0..31 x columns 32..63, which
// no read touches) by gathering from the record's 16x16 blocks; units above the
// diagonal read the record's zero bytes.

// Workgroup: NW waves, each owning 16 state rows v0 + 16 w .. of one (sequence, v-head)
// for all 128 columns; the waves share the chunk's K, Q, V, T', P' through LDS and
// never exchange state. Per chunk and wave (state S0 at chunk start, T' = T diag(beta)):
//   X  = K S0^T                      (S0 as bf16 hi + lo)
//   R  = V - gamma X
//   U  = T' R                        (T', R as hi + lo; three products)
//   O  = scale gamma Q S0^T + P' U   (S0 hi, U bf16)
//   S  = gammaC S0 + (dec U)^T K     (dec U as hi + lo)
// Row orders inside a 32-row block are permuted so that every MFMA result is already
// the next MFMA's operand: X and U tiles use token rows 32 (tt/2) + 8 (m/4) + 4 (tt%2)
// + m%4, state tiles kt = 2s + h hold columns 32 s + 8 (m/4) + 4 h + m%4. K^T and the
// V columns are read with the LDS transpose read.
// SEG: the grid walks segment jobs (p.jobs); otherwise whole sequences, and none of the
// segment code is compiled in (it costs the whole-sequence loop registers).
template <int NW, bool SEG>
__device__ __forceinline__ void scan_body(const ScanArgs &p, ScanBuf<NW> &BA, ScanBuf<NW> &BB)
{
    constexpr int TPH = 8 / NW;  // workgroups per (sequence, v-head)
    // Workgroups of one (sequence, q/k head) share K, Q through L2: one XCD for them all
    // (workgroup ids are dealt to the 8 XCDs round-robin).
    const int pid = blockIdx.x, xcd = pid & 7, slot = pid >> 3;
    const int gsz = TPH * p.ratio;
    const int wi = slot % gsz;
    const int grp = (slot / gsz) * 8 + xcd;
    if (grp >= p.ngroups)
        return;
    int n, kind = kJobFirst, cb = 0, ce = 0x7fffffff, q = -1, steps = 0, last = 0;
    if constexpr (SEG) {
        const int e = grp / p.HQK;
        if (e >= p.header[p.njob_idx])
            return;
        const int32_t *je = p.jobs + 8 * (p.job_first + e);
        n = je[0];
        kind = je[1];
        cb = je[2];
        ce = je[3];
        q = je[4];
        steps = je[5];
        last = je[6];
    } else {
        n = p.seq_order[grp / p.HQK];
    }
    const int g = grp % p.HQK;
    const int h = g * p.ratio + wi / TPH;
    const int v0 = (wi % TPH) * 16 * NW;
    const int tok0 = p.seq_tok0[n], len = p.seq_len[n], c0 = p.seq_chunk0[n];
    // records exist only for chunk ids < header[0] (see the plan kernel's clamp)
    const int nck = min((len + kC - 1) / kC, max(p.header[0] - c0, 0));
    ce = min(ce, nck);
    const bool do_out = kind == kJobFirst || kind == kJobResume;
    const bool vzero = kind == kJobIdent;

    // w is wave-uniform: LDS copy destinations (M0) are then scalar arithmetic
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63,
              lr = l & 15, lg = l >> 4;
    const int v0w = v0 + 16 * w;

    // ---- copy plan. Every copy is a buffer load straight to LDS; per-lane source offsets
    // are chunk-invariant and computed once. Rows past a chunk's end fall outside the
    // chunk's buffer range and read as zero: those rows meet beta = 0 or the causal mask
    // only, and their outputs are never stored.
    const uint32_t kst2 = (uint32_t)p.k_st * 2, qst2 = (uint32_t)p.q_st * 2;
    const uint32_t vst2 = (uint32_t)p.v_st * 2, ost2 = (uint32_t)p.o_st * 2;
    const char *kbase = (const char *)(p.k + (int64_t)tok0 * p.k_st + g * p.k_sh);
    const char *qbase = (const char *)(p.q + (int64_t)tok0 * p.q_st + g * p.q_sh);
    const char *vbase = (const char *)(p.v + (int64_t)tok0 * p.v_st + h * p.v_sh + v0);
    char *obase = (char *)(p.out + (int64_t)tok0 * p.o_st + h * p.o_sh + v0w);
    const int64_t kstep = (int64_t)kC * p.k_st * 2, qstep = (int64_t)kC * p.q_st * 2;
    const int64_t vstep = (int64_t)kC * p.v_st * 2, ostep = (int64_t)kC * p.o_st * 2;
    const char *rbase = p.records + ((int64_t)c0 * p.HV + h) * kRecBytes;
    const int64_t rstep = (int64_t)p.HV * kRecBytes;

    constexpr int VWIN = 2 * NW;               // V windows
    constexpr int NWIN = 32 + VWIN + 19;       // all windows
    constexpr int PER = (NWIN + NW - 1) / NW;  // windows per wave

    // Source offset of this lane in window i (compile-time) of this wave; window kinds
    // follow win = w + NW i: K rows 4b..4b+3 (16 windows), Q (16), V (NW == 8: 4 rows per
    // window, NW == 4: 8 rows), then 18 T' / P' windows and the gate area.
    uint32_t woff[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int win = w + NW * i;
        uint32_t off = 0;
        if (NW * i < 16) {
            const int t = 4 * win + (l >> 4), cs = l & 15;
            off = (uint32_t)t * kst2 + 16u * (cs ^ kswz(t));
        } else if (NW * i < 32) {
            const int t = 4 * (win - 16) + (l >> 4), cs = l & 15;
            off = (uint32_t)t * qst2 + 16u * (cs ^ (t & 15));
        } else if (NW * i < 32 + VWIN) {
            const int b = win - 32;
            const int t = NW == 8 ? 4 * b + (l >> 4) : 8 * b + (l >> 3);
            const int cs = NW == 8 ? (l & 15) : (l & 7);
            off = (uint32_t)t * vst2 + 16u * (cs ^ (2 * (t & 3)));
        } else {
            const int r = win - 32 - VWIN;
            if (r < 18) {
                const int mt = r / 6, pr = r % 6, b = pr == 0 ? 0 : (pr == 1 ? 2 : pr + 2);
                const int u = 64 * b + l;  // this lane's LDS unit
                const int row = mt < 2 ? tlay_row(u) : play_row(u), cc = lay_col(u);
                const int bi = row >> 4, bj = cc >> 1;
                const int mbase = mt == 0 ? kRecThi : (mt == 1 ? kRecTlo : kRecP);
                off = bj <= bi ? (uint32_t)(mbase + (tri_blk(bi, bj) * 32 + 2 * (row & 15) + (cc & 1)) * 16)
                               : (uint32_t)kRecZero;
            } else {
                off = kRecGates + 16u * l;
            }
        }
        woff[i] = off;
    }

    // Buffer ranges of chunk c: K / Q / V end after the chunk's last row.
    struct ChunkSrc {
        __amdgpu_buffer_rsrc_t k, q, v, r;
    };
    // (valid == false: empty ranges, every copy writes zeros and reads nothing)
    auto chunk_src_v = [&](int c, bool valid) {
        const int lenc = min(kC, len - c * kC);
        ChunkSrc cs;
        cs.k = __builtin_amdgcn_make_buffer_rsrc((void *)(kbase + c * kstep), 0,
                                                 valid ? (int)((uint32_t)(lenc - 1) * kst2 + 256u) : 0, 0x00020000);
        cs.q = __builtin_amdgcn_make_buffer_rsrc((void *)(qbase + c * qstep), 0,
                                                 valid ? (int)((uint32_t)(lenc - 1) * qst2 + 256u) : 0, 0x00020000);
        cs.v = __builtin_amdgcn_make_buffer_rsrc((void *)(vbase + c * vstep), 0,
                                                 valid ? (int)((uint32_t)(lenc - 1) * vst2 + 32u * NW) : 0, 0x00020000);
        cs.r = __builtin_amdgcn_make_buffer_rsrc((void *)(rbase + c * rstep), 0, valid ? kRecBytes : 0, 0x00020000);
        return cs;
    };
    auto chunk_src = [&](int c) { return chunk_src_v(c, true); };
    auto issue_win = [&](ScanBuf<NW> &B, const ChunkSrc &cs, const int i) {
        const int win = w + NW * i;  // window kind is a compile-time function of i
        if (NW * i < 16) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(cs.k, (GDN_LDS void *)&B.K[64 * win], 16, woff[i], 0, 0, 0);
        } else if (NW * i < 32) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(cs.q, (GDN_LDS void *)&B.Q[64 * (win - 16)], 16, woff[i], 0, 0, 0);
        } else if (NW * i < 32 + VWIN) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(cs.v, (GDN_LDS void *)&B.V[64 * (win - 32)], 16, woff[i], 0, 0, 0);
        } else if (win < NWIN) {
            const int r = win - 32 - VWIN;
            if (r < 18) {
                const int mt = r / 6, pr = r % 6, b = pr == 0 ? 0 : (pr == 1 ? 2 : pr + 2);
                u32x4 *dst = mt == 2 ? &B.P[64 * b] : &B.T[mt][64 * b];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(cs.r, (GDN_LDS void *)dst, 16, woff[i], 0, 0, 0);
            } else {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(cs.r, (GDN_LDS void *)&B.G[0], 16, woff[i], 0, 0, 0);
            }
        }
    };
    auto issue_chunk = [&](ScanBuf<NW> &B, int c) {
        const ChunkSrc cs = chunk_src(c);
#pragma unroll
        for (int i = 0; i < PER; ++i)
            issue_win(B, cs, i);
    };

    // ---- LDS read offsets (bytes within a ScanBuf member; chunk-invariant)
    const int c_ = lr & 3, r_ = lr >> 2;
    uint32_t koffA[4], ktoff[4], qoff[4];
    const int ta = 8 * (lr >> 2) + (lr & 3), tk = 8 * lg + r_;  // rows of the K and K^T reads
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        koffA[s] = 16u * (16 * ta + ((4 * s + lg) ^ kswz(ta)));
        ktoff[s] = 256u * tk + 16u * ((4 * s + c_) ^ kswz(tk));
        qoff[s] = 16u * (16 * lr + ((4 * s + lg) ^ lr));
    }
    const uint32_t voff = 32u * NW * (8 * lg + r_) + 16u * ((2 * w + (c_ >> 1)) ^ (2 * r_)) + 8u * (c_ & 1);
    // T' / P' operand of tile tt, k-step sp: byte tpoff + 2048 tt + 1024 sp
    const uint32_t tpoff = 16u * (lr & 7) + 128u * (lg & 1) + 256u * (lr >> 3) + 512u * (lg >> 1);
    const uint32_t goff = 32u * lg, sgoff = 4u * lr;

    // this lane's units of a slot in register-image order: S[t] at + 256 t
    auto seg_img = [&](const float *base, int qs) {
        return base + ((int64_t)qs * p.HV + h) * kSlotFloats + ((v0w >> 4) * 8 * 64 + l) * 4;
    };
    // A resumed segment with chain steps first issues the first step's M^T copy (into BB,
    // which no chunk copy touches before the loop) and R loads, then the first chunk's copies.
    const bool chain = SEG && steps > 0;
    u32x4 *mb = (u32x4 *)&BB;
    static_assert(sizeof(ScanBuf<NW>) >= 2 * kMtUnits * 16, "M^T must fit one chunk buffer");
    constexpr int MWIN = 2 * kMtUnits / 64 / NW;  // 1 KB windows per wave
    auto issue_m = [&](int qs) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(p.seg_mt + ((int64_t)qs * p.HV + h) * kSlotFloats), 0, 2 * kMtUnits * 16, 0x00020000);
#pragma unroll
        for (int i = 0; i < MWIN; ++i) {
            const int b = w + NW * i;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (GDN_LDS void *)&mb[64 * b], 16,
                                                     16u * (uint32_t)(64 * b + l), 0, 0, 0);
        }
    };
    f32x4 R[8];
    auto load_r = [&](int qs) {
        const float *rp = seg_img(p.seg_r, qs);
#pragma unroll
        for (int t = 0; t < 8; ++t)
            R[t] = *(const f32x4 *)(rp + 256 * t);
    };
    if (chain) {
        issue_m(q);
        load_r(q);
        // unconditional, so the number of operations in flight is the same on every path
        const ChunkSrc cs = chunk_src_v(cb, ce > cb);
#pragma unroll
        for (int i = 0; i < PER; ++i)
            issue_win(BA, cs, i);
    } else if (ce > cb) {
        issue_chunk(BA, cb);
    }

    // ---- state: S[2 s + h] holds S[v0w + lr][32 s + 8 lg + 4 h + i], i = 0..3
    f32x4 S[8];
    // (branch on workgroup-uniform flags: a test of the per-lane pointers would make the
    // compiler wait for each load before the next)
    if (SEG && kind == kJobResume) {
        const float *ip = seg_img(p.seg_sin, q);
#pragma unroll
        for (int t = 0; t < 8; ++t)
            S[t] = *(const f32x4 *)(ip + 256 * t);
    } else if (kind == kJobFirst && p.state) {
        const float *sp = p.state + n * p.st_sn + h * p.st_sh + (int64_t)(v0w + lr) * p.st_sv + 8 * lg;
#pragma unroll
        for (int t = 0; t < 8; ++t)
            S[t] = *(const f32x4 *)(sp + 32 * (t >> 1) + 4 * (t & 1));
    } else {
        const bool ident = SEG && kind == kJobIdent;  // row v0w + lr of the identity
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                S[t][i] = ident && 32 * (t >> 1) + 8 * lg + 4 * (t & 1) + i == v0w + lr ? 1.f : 0.f;
    }

    // ---- chain steps of a resumed segment: S <- S M_m + R_m for the slots q .. q + steps - 1.
    // Row-wise this is S^T <- M_m^T S^T + R_m^T: an MFMA with A = M_m^T from LDS and B = the
    // wave's own state rows, whose C layout is again the state layout (output tile t covers
    // columns j(m) = 32 (t / 2) + 8 (m / 4) + 4 (t % 2) + m % 4). M_m and S are split into
    // bf16 hi + lo (three products) so the chained state keeps fp32 accuracy. M_m^T is
    // copied unit by unit into BB, which no chunk copy touches before the loop starts;
    // LDS unit 16 j + (cu ^ kswz(j)) holds row j, k-chunk cu (the K layout of the loop).
    if (chain) {
        for (int m = 0; m < steps; ++m) {
            if (m == 0) {
                // M_q^T and R_q are in (memory operations complete in order); the first
                // chunk's copies, at least NWIN / NW per wave, may still be in flight
                constexpr int nv = NWIN / NW;
                static_assert(nv < 64, "vmcnt range");
                __builtin_amdgcn_s_waitcnt((nv & 15) | ((nv >> 4) << 14) | 0x0f70);
                lds_barrier_inflight();
            } else {
                dma_barrier();  // M_m^T is in LDS, R_m in registers
            }
            u32x4 Bh[4], Bl[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
                split_bf16x2(S[2 * ks][0], S[2 * ks][1], h0, l0);
                split_bf16x2(S[2 * ks][2], S[2 * ks][3], h1, l1);
                split_bf16x2(S[2 * ks + 1][0], S[2 * ks + 1][1], h2, l2);
                split_bf16x2(S[2 * ks + 1][2], S[2 * ks + 1][3], h3, l3);
                Bh[ks] = u32x4{h0, h1, h2, h3};
                Bl[ks] = u32x4{l0, l1, l2, l3};
            }
            auto read_a = [&](int t, u32x4 *Ah, u32x4 *Al) {
                const int j = 32 * (t >> 1) + 8 * (lr >> 2) + 4 * (t & 1) + (lr & 3), sw = kswz(j);
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int u = 16 * j + ((4 * ks + lg) ^ sw);
                    Ah[ks] = mb[u];
                    Al[ks] = mb[kMtUnits + u];
                }
            };
            u32x4 Ah[2][4], Al[2][4];
            read_a(0, Ah[0], Al[0]);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                __builtin_amdgcn_sched_barrier(0);
                if (t < 7)
                    read_a(t + 1, Ah[(t + 1) & 1], Al[(t + 1) & 1]);
                f32x4 acc = R[t];
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    acc = mfma_bf16(Ah[t & 1][ks], Bh[ks], acc);
                    acc = mfma_bf16(Ah[t & 1][ks], Bl[ks], acc);
                    acc = mfma_bf16(Al[t & 1][ks], Bh[ks], acc);
                }
                S[t] = acc;
            }
            __builtin_amdgcn_sched_barrier(0);
            if (m + 1 < steps) {
                lds_barrier_inflight();  // every wave is done with M_m^T
                issue_m(q + m + 1);
                load_r(q + m + 1);
            }
        }
    }

    // Operand reads run one step ahead of the MFMAs that consume them; sched_barrier
    // keeps each step's reads, VALU work and MFMAs in the order written.
    // The next chunk's copies (PER windows) are spread over phases (a) and (c): issued
    // all at once they queue behind each other and stall the issuing waves.
    auto compute = [&](ScanBuf<NW> &B, int c, ScanBuf<NW> &Bn, bool more) {
        const int lenc = min(kC, len - c * kC);
        const ChunkSrc ncs = chunk_src(more ? c + 1 : c);
        auto dma_at = [&](const int slot) {  // slots 0..7: after (a) steps 0..3, (c) tiles 0..3
#pragma unroll
            for (int i = 0; i < PER; ++i)
                if ((i * 8) / PER == slot && more)
                    issue_win(Bn, ncs, i);
        };
        const char *Kb = (const char *)B.K, *Qb = (const char *)B.Q, *Vb = (const char *)B.V;
        const char *Th = (const char *)B.T[0], *Tl = (const char *)B.T[1];
        const char *Pb = (const char *)B.P, *Gb = (const char *)B.G;
        auto kA = [&](int s, int tt) {
            return *(const u32x4 *)(Kb + koffA[s] + 256 * (32 * (tt >> 1) + 4 * (tt & 1)));
        };
        auto split_s = [&](int s, u32x4 &bh, u32x4 &bl) {
            uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
            split_bf16x2(S[2 * s][0], S[2 * s][1], h0, l0);
            split_bf16x2(S[2 * s][2], S[2 * s][3], h1, l1);
            split_bf16x2(S[2 * s + 1][0], S[2 * s + 1][1], h2, l2);
            split_bf16x2(S[2 * s + 1][2], S[2 * s + 1][3], h3, l3);
            bh = u32x4{h0, h1, h2, h3};
            bl = u32x4{l0, l1, l2, l3};
        };

        // (a) S0 as MFMA operands (hi + lo), X = K S0^T
        u32x4 Bh[4], Bl[4], ka[2][4];
        f32x4 X[4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            ka[0][tt] = kA(0, tt);
            X[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        split_s(0, Bh[0], Bl[0]);
        u32x2 vv[4];
        f32x4 gm[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            __builtin_amdgcn_sched_barrier(0);
            if (s < 3) {
#pragma unroll
                for (int tt = 0; tt < 4; ++tt)
                    ka[(s + 1) & 1][tt] = kA(s + 1, tt);
                split_s(s + 1, Bh[s + 1], Bl[s + 1]);
            } else {
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {  // (b)'s operands
                    const int trow = 32 * (tt >> 1) + 4 * (tt & 1);
                    vv[tt] = lds_tr16(Vb + voff + 32 * NW * trow);
                    if (vzero)
                        vv[tt] = u32x2{0u, 0u};
                    gm[tt] = *(const f32x4 *)(Gb + goff + 4 * trow);
                }
            }
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                X[tt] = mfma_bf16(ka[s & 1][tt], Bh[s], X[tt]);
                X[tt] = mfma_bf16(ka[s & 1][tt], Bl[s], X[tt]);
            }
            dma_at(s);
        }
        __builtin_amdgcn_sched_barrier(0);

        // (b) R = V - gamma X -> operands (hi + lo) over token blocks s'
        u32x4 Rh[2], Rl[2];
        auto tRead = [&](int tt, int sp, u32x4 &th, u32x4 &tl) {
            const uint32_t o = tpoff + 2048 * tt + 1024 * sp;
            th = *(const u32x4 *)(Th + o);
            tl = *(const u32x4 *)(Tl + o);
        };
        u32x4 tA[2][2][2];  // [buffer][sp][hi / lo]
        tRead(0, 0, tA[0][0][0], tA[0][0][1]);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const float r0 = fmaf(-gm[tt][0], X[tt][0], bf16lo(vv[tt][0]));
            const float r1 = fmaf(-gm[tt][1], X[tt][1], bf16hi(vv[tt][0]));
            const float r2 = fmaf(-gm[tt][2], X[tt][2], bf16lo(vv[tt][1]));
            const float r3 = fmaf(-gm[tt][3], X[tt][3], bf16hi(vv[tt][1]));
            uint32_t h01, l01, h23, l23;
            split_bf16x2(r0, r1, h01, l01);
            split_bf16x2(r2, r3, h23, l23);
            const int e = 2 * (tt & 1);
            Rh[tt >> 1][e] = h01; Rh[tt >> 1][e + 1] = h23;
            Rl[tt >> 1][e] = l01; Rl[tt >> 1][e + 1] = l23;
        }

        // (c) U = T' R
        f32x4 U[4];
        f32x4 dc[4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            __builtin_amdgcn_sched_barrier(0);
            const int cb = tt & 1;
            if (tt < 3) {  // next tile's T' blocks
#pragma unroll
                for (int sp = 0; sp <= ((tt + 1) >> 1); ++sp)
                    tRead(tt + 1, sp, tA[cb ^ 1][sp][0], tA[cb ^ 1][sp][1]);
            } else {
#pragma unroll
                for (int t2 = 0; t2 < 4; ++t2)  // (d)'s operands
                    dc[t2] = *(const f32x4 *)(Gb + 256 + goff + 4 * (32 * (t2 >> 1) + 4 * (t2 & 1)));
            }
            U[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sp = 0; sp <= (tt >> 1); ++sp) {
                U[tt] = mfma_bf16(tA[cb][sp][0], Rh[sp], U[tt]);
                U[tt] = mfma_bf16(tA[cb][sp][0], Rl[sp], U[tt]);
                U[tt] = mfma_bf16(tA[cb][sp][1], Rh[sp], U[tt]);
            }
            dma_at(4 + tt);
        }
        __builtin_amdgcn_sched_barrier(0);

        // (d) W = dec U (hi + lo) for the state update, U (bf16) for the readout
        auto qRead = [&](int tt, u32x4 *qv, u32x4 *pv) {
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2)
                qv[s2] = *(const u32x4 *)(Qb + qoff[s2] + 4096 * tt);
#pragma unroll
            for (int sp = 0; sp <= (tt >> 1); ++sp)
                pv[sp] = *(const u32x4 *)(Pb + tpoff + 2048 * tt + 1024 * sp);
        };
        u32x4 qA[2][4], pA[2][2];
        qRead(0, qA[0], pA[0]);
        u32x4 Wh[2], Wl[2], Ub[2];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            uint32_t h01, l01, h23, l23;
            split_bf16x2(dc[tt][0] * U[tt][0], dc[tt][1] * U[tt][1], h01, l01);
            split_bf16x2(dc[tt][2] * U[tt][2], dc[tt][3] * U[tt][3], h23, l23);
            const uint32_t u01 = pack_bf16x2(U[tt][0], U[tt][1]), u23 = pack_bf16x2(U[tt][2], U[tt][3]);
            const int e = 2 * (tt & 1);
            Wh[tt >> 1][e] = h01; Wh[tt >> 1][e + 1] = h23;
            Wl[tt >> 1][e] = l01; Wl[tt >> 1][e + 1] = l23;
            Ub[tt >> 1][e] = u01; Ub[tt >> 1][e + 1] = u23;
        }

        // (e) O^T = scale gamma S0 Q^T + U^T P'^T; lane (t = 16 tt + lr) stores 4 values.
        // Rows past the chunk's end fall outside the buffer range and are dropped.
        const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
            obase + c * ostep, 0, (int)((uint32_t)lenc * ost2), 0x00020000);
        auto ktRead = [&](int gidx, u32x4 *ko) {
            const int s2 = gidx >> 1, hh = gidx & 1;
#pragma unroll
            for (int sp = 0; sp < 2; ++sp) {
                const u32x2 k0 = lds_tr16(Kb + ktoff[s2] + 256 * (32 * sp) + 8 * hh);
                const u32x2 k1 = lds_tr16(Kb + ktoff[s2] + 256 * (32 * sp + 4) + 8 * hh);
                ko[sp] = u32x4{k0[0], k0[1], k1[0], k1[1]};
            }
        };
        u32x4 kt[2][2];
        if (!do_out)
            ktRead(0, kt[0]);  // (f)'s first operands
        // Tile tt's combine and store run after tile tt + 1's MFMAs are issued, so they
        // never wait on the MFMA chain that produced them.
        f32x4 Oi[2], Oa[2];
        float sg[2];
        auto out_epi = [&](int tt) {
            const int cb = tt & 1;
            const uint32_t o01 = pack_bf16x2(fmaf(sg[cb], Oi[cb][0], Oa[cb][0]), fmaf(sg[cb], Oi[cb][1], Oa[cb][1]));
            const uint32_t o23 = pack_bf16x2(fmaf(sg[cb], Oi[cb][2], Oa[cb][2]), fmaf(sg[cb], Oi[cb][3], Oa[cb][3]));
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{o01, o23}, orsrc,
                                                  (int)((uint32_t)(16 * tt + lr) * ost2 + 8u * lg), 0, 0);
        };
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            if (!do_out)
                break;
            __builtin_amdgcn_sched_barrier(0);
            const int cb = tt & 1;
            if (tt < 3)
                qRead(tt + 1, qA[cb ^ 1], pA[cb ^ 1]);
            else
                ktRead(0, kt[0]);  // (f)'s first operands
            sg[cb] = *(const float *)(Gb + 512 + sgoff + 64 * tt);
            Oi[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
            Oa[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2)
                Oi[cb] = mfma_bf16(Bh[s2], qA[cb][s2], Oi[cb]);
#pragma unroll
            for (int sp = 0; sp <= (tt >> 1); ++sp)
                Oa[cb] = mfma_bf16(Ub[sp], pA[cb][sp], Oa[cb]);
            if (tt > 0)
                out_epi(tt - 1);
        }

        // (f) S = gammaC S0 + W^T K
        const float gC = *(const float *)(Gb + 768);
#pragma unroll
        for (int gidx = 0; gidx < 8; ++gidx) {
            __builtin_amdgcn_sched_barrier(0);
            if (gidx < 7)
                ktRead(gidx + 1, kt[(gidx + 1) & 1]);
            f32x4 acc = gC * S[gidx];
#pragma unroll
            for (int sp = 0; sp < 2; ++sp) {
                acc = mfma_bf16(kt[gidx & 1][sp], Wh[sp], acc);
                acc = mfma_bf16(kt[gidx & 1][sp], Wl[sp], acc);
            }
            if (gidx == 0 && do_out)
                out_epi(3);
            S[gidx] = acc;
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    for (int c = cb; c < ce; c += 2) {
        dma_barrier();  // chunk c is in BA; every wave is done with BB
        compute(BA, c, BB, c + 1 < ce);
        if (c + 1 >= ce)
            break;
        dma_barrier();
        compute(BB, c + 1, BA, c + 2 < ce);
    }

    if (SEG && kind == kJobResume && !last)
        return;
    if (SEG && kind == kJobIdent) {
        // This wave holds rows k = v0w .. v0w + 15 of M_s, i.e. k-chunks cu0 and cu0 + 1 of
        // every row j of M_s^T. Transpose them through a per-wave LDS stage (fp32, row j at
        // 64 j bytes) in the chunk buffer the last chunk did not use (free since the last
        // chunk's barrier), then write each unit split into bf16 hi and lo; the two units of
        // one j are adjacent (cu0 is even), so lane pairs write 32 contiguous bytes.
        float *stg = (float *)(((ce - cb) & 1) ? (void *)&BB : (void *)&BA) + 2048 * w;
        static_assert(sizeof(ScanBuf<NW>) >= NW * 2048 * 4, "stage must fit one chunk buffer");
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    stg[(32 * s + 8 * lg + 4 * hh + i) * 16 + lr] = S[2 * s + hh][i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        u32x4 *mt = (u32x4 *)(p.seg_mt + ((int64_t)q * p.HV + h) * kSlotFloats);
        const int cu0 = v0w >> 3;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int u = l + 64 * r, j = u >> 1, c2 = u & 1;
            const f32x4 a = *(const f32x4 *)(stg + 16 * j + 8 * c2);
            const f32x4 b = *(const f32x4 *)(stg + 16 * j + 8 * c2 + 4);
            uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
            split_bf16x2(a[0], a[1], h0, l0);
            split_bf16x2(a[2], a[3], h1, l1);
            split_bf16x2(b[0], b[1], h2, l2);
            split_bf16x2(b[2], b[3], h3, l3);
            const int un = 16 * j + ((cu0 + c2) ^ kswz(j));
            mt[un] = u32x4{h0, h1, h2, h3};
            mt[kMtUnits + un] = u32x4{l0, l1, l2, l3};
        }
        return;
    }
    if (SEG && (kind == kJobZero || (kind == kJobFirst && q >= 0))) {  // R_s or S_in(1)
        float *ip = (float *)seg_img(kind == kJobZero ? p.seg_r : p.seg_sin, q);
#pragma unroll
        for (int t = 0; t < 8; ++t)
            *(f32x4 *)(ip + 256 * t) = S[t];
        return;
    }
    float *np = p.new_state + n * p.ns_sn + h * p.ns_sh + (int64_t)(v0w + lr) * p.ns_sv + 8 * lg;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        *(f32x4 *)(np + 32 * s) = S[2 * s];
        *(f32x4 *)(np + 32 * s + 4) = S[2 * s + 1];
    }
}

template <bool SEG>
__global__ __launch_bounds__(512) void gdn_prefill_scan8_kernel(ScanArgs p)
{
    __shared__ ScanBuf<8> bufA, bufB;
    scan_body<8, SEG>(p, bufA, bufB);
}

template <bool SEG>
__global__ __launch_bounds__(256) void gdn_prefill_scan4_kernel(ScanArgs p)
{
    __shared__ ScanBuf<4> bufA, bufB;
    scan_body<4, SEG>(p, bufA, bufB);
}

}  // namespace gdn

// ------------------------------------------------------------------------- host side
namespace {

constexpr int64_t kChunkH = 64;
constexpr int kZeroFillBlocks = 64;

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

int64_t max_chunks(int64_t T, int64_t N) { return (T + kChunkH - 1) / kChunkH + N; }

// Segments per sequence (the default variant only): when (sequence, v-head) pairs are too
// few to fill 256 CUs, the largest G <= 8 whose pass-A jobs N HV (2 G - 3) still fit one
// workgroup per CU; 1 means no segments (G = 2 would scan its halves one after the other).
int seg_count(int64_t T, int64_t N, int64_t HV)
{
    if (T <= 0 || N <= 0 || N * HV * 3 > 256)
        return 1;
    int G = 3;
    while (G < 8 && N * HV * (2 * (G + 1) - 3) <= 256)
        ++G;
    return G;
}

struct Layout {
    int64_t nc;
    int64_t header, chunk_tok0, chunk_len, seq_chunk0, seq_order, seq_tok0, seq_len, records,
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
    L.seq_order = o;
    o += N * 4;
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
        o = L.jobs + (L.capA + L.capC) * 8 * 4;
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
    pa.seq_order = (int32_t *)(ws + L.seq_order);
    pa.seq_tok0 = (int32_t *)(ws + L.seq_tok0);
    pa.seq_len = (int32_t *)(ws + L.seq_len);
    pa.out = (gdn::bf16_t *)p->output;
    pa.o_st = p->output_stride[0];
    pa.o_sh = p->output_stride[1];
    // segments only for the default variant (the tuning variants keep whole sequences)
    const int G = p->variant == 0 ? L.G : 1;
    pa.seg_G = G;
    pa.seg_capA = (int)L.capA;
    pa.jobs = G > 1 ? (int32_t *)(ws + L.jobs) : nullptr;
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
        sa.seq_order = pa.seq_order;
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
            rc = scan(L.capA, false);
            if (rc)
                return rc;
            // pass C: outputs of segments 1 .. G - 1, each chaining its entering state first;
            // the last segment's final state is new_state
            sa.job_first = (int)L.capA;
            sa.njob_idx = 2;
            rc = scan(L.capC, L.capC * HV <= 128);
        } else {
            const bool nw4 = p->variant == 1 || (p->variant != 2 && (int64_t)N * HV <= 128);
            rc = scan(N, nw4);
        }
        if (rc)
            return rc;
    }
    return GDN_OK;
}
