// Prefill plan kernel (more than 64 sequences): sequence -> chunk tables from cu_seqlens on
// the device, longest-first sequence order, zero-fill of rows outside every sequence.
#include "gdn_prefill.h"

namespace gdn {

__global__ __launch_bounds__(256) void gdn_prefill_plan_kernel(PlanArgs p)
{
    const int tid = threadIdx.x;
    if (blockIdx.x == 0) {
        // Chunk counts are clamped so that malformed (non-monotone) cu_seqlens can
        // never index past the chunk tables or records sized for nc chunks; for
        // valid input sum(ceil(len / C)) <= ceil(T / C) + N = nc always holds.
        __shared__ int64_t s_wtot[4];  // per-wave totals of the block scan
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
            // inclusive prefix sum over the block: DPP inside each wave, then the totals
            // of the waves before this one
            int64_t incl = wave_prefix_sum_i64(nck);
            if ((tid & 63) == 63)
                s_wtot[tid >> 6] = incl;
            __syncthreads();
            for (int w2 = 0; w2 < (tid >> 6); ++w2)
                incl += s_wtot[w2];
            const int64_t first = s_carry + incl - nck;
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
                    // too many sequences to sort: identity order
                    *(int4 *)(p.seq_rank + 4 * n) =
                        int4{n, t0, ln, (int32_t)(first < p.nc ? first : p.nc)};
                }
            }
            __syncthreads();  // every lane has read s_carry and s_wtot
            if (tid == 255)
                s_carry += incl;
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
        // Longest-first order (identity when N is large, written above).
        if (par) {
            for (int n = tid; n < p.N; n += 256) {
                const int mine = s_nck[n];
                int rank = 0;
                for (int m = 0; m < p.N; ++m) {
                    const int o = s_nck[m];
                    rank += (o > mine) || (o == mine && m < n);
                }
                *(int4 *)(p.seq_rank + 4 * rank) = int4{n, s_t0[n], s_len[n], s_first[n]};
            }
        }
        // (segment job tables come from the prep kernel: segments are used up to 64
        // sequences only, where the prep kernel plans for itself)
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

}  // namespace gdn
