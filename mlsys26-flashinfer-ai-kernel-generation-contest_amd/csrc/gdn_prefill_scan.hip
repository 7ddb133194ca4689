// Prefill scan kernels: the sequential chunk recurrence, state in registers, for whole
// sequences or segment jobs.
#include "gdn_prefill.h"

namespace gdn {

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
// A scan workgroup's job: its (sequence or segment job, q/k head) group grp, its place wi
// among the group's workgroups, and the job's sequence, kind and chunk range.
struct ScanJob {
    int grp, wi, n, tok0, len, c0, kind, cb, ce, q, steps, last;
};

// Finds this workgroup's job (SEG: in the segment job table); false when it has none.
template <int NW, bool SEG>
__device__ __forceinline__ bool scan_job(const ScanArgs &p, ScanJob &j)
{
    constexpr int TPH = 8 / NW;  // workgroups per (sequence, v-head)
    // Workgroups of one (sequence, q/k head) share K, Q through L2: one XCD for them all
    // (workgroup ids are dealt to the 8 XCDs round-robin).
    const int pid = blockIdx.x, xcd = pid & 7, slot = pid >> 3;
    const int gsz = TPH * p.ratio;
    j.wi = slot % gsz;
    j.grp = (slot / gsz) * 8 + xcd;
    if (j.grp >= p.ngroups)
        return false;
    j.kind = kJobFirst;
    j.cb = 0;
    j.ce = 0x7fffffff;
    j.q = -1;
    j.steps = 0;
    j.last = 0;
    if constexpr (SEG) {
        // the grid covers the job table's capacity, so the entry exists even past the job
        // count, and both load together
        const int e = j.grp / p.HQK;
        const int4 *je = (const int4 *)(p.jobs + kJobInts * (p.job_first + e));
        const int4 j0 = je[0], j1 = je[1], j2 = je[2];
        if (e >= p.header[p.njob_idx])
            return false;
        j.n = j0.x;
        j.kind = j0.y;
        j.cb = j0.z;
        j.ce = j0.w;
        j.q = j1.x;
        j.steps = j1.y;
        j.last = j1.z;
        j.tok0 = j1.w;
        j.len = j2.x;
        j.c0 = j2.y;
    } else {
        // ranks below ngroups / HQK = N all have an entry: load it with the count
        const int e = j.grp / p.HQK;
        const int4 r = *(const int4 *)(p.seq_rank + 4 * e);
        if (p.njob_idx > 0 && e >= p.header[p.njob_idx])
            return false;
        j.n = r.x;
        j.tok0 = r.y;
        j.len = r.z;
        j.c0 = r.w;
    }
    return true;
}

// SEG: the body handles every segment job kind; otherwise only jobs from the initial state
// with outputs into new_state (whole sequences), with none of the segment code compiled in.
// OUTS (segment bodies): 1 compiles the body for jobs with outputs (kJobFirst, kJobResume),
// 0 for value-row maps (kJobZero), 2 for identity-row maps (kJobIdent), so the loop carries
// no run-time test of the job kind. The maps copy neither Q nor P' (no outputs), and the
// identity maps no V (V = 0).
// INST tags an instance: the whole-sequence body inside a segment kernel is instance 1, so
// each instance is used by one kernel only (hipcc's host pass rejects a second kernel's use
// of an instance of this device-only template: "substitution failure").
template <int NW, bool SEG, int INST = 0, int OUTS = -1>
__device__ __forceinline__ void scan_body(const ScanArgs &p, const ScanJob &job, ScanBuf<NW> &BA,
                                          ScanBuf<NW> &BB)
{
    constexpr int TPH = 8 / NW;  // workgroups per (sequence, v-head)
    const int grp = job.grp, wi = job.wi, n = job.n, tok0 = job.tok0, len = job.len,
              c0 = job.c0, kind = SEG ? job.kind : kJobFirst, cb = SEG ? job.cb : 0,
              q = SEG ? job.q : -1, steps = SEG ? job.steps : 0, last = SEG ? job.last : 0;
    int ce = SEG ? job.ce : 0x7fffffff;
    const int g = grp % p.HQK;
    const int h = g * p.ratio + wi / TPH;
    const int v0 = (wi % TPH) * 16 * NW;
    // records exist only for chunk ids < header[0] (see the plan kernel's clamp)
    const int nck = min((len + kC - 1) / kC, max(p.header[0] - c0, 0));
    ce = min(ce, nck);
    const bool do_out = OUTS >= 0 ? OUTS == 1 : kind == kJobFirst || kind == kJobResume;
    const bool vzero = OUTS == 2 || (OUTS < 0 && kind == kJobIdent);

    // w is wave-uniform: LDS copy destinations (M0) are then scalar arithmetic
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63,
              lr = l & 15, lg = l >> 4;
    const int v0w = v0 + 16 * w;

    // Every bf16 hi / lo split of the loop. With one wave per SIMD (NW == 4) a wave issues
    // alone and each VALU instruction it saves counts: the dot-product residual, with gammaC
    // S0 formed early (phase (a) below), saves 64 of ~330 a chunk (qk4_v8 batches of whole
    // sequences 4-6 % faster on MI355X). With two waves per SIMD the 8-wave scan ran no
    // faster with it (1-2 % slower with the early gammaC S0), so it keeps the plain split.
    SplitConsts sk{};
    if constexpr (NW == 4)
        sk = split_consts();
    auto split2 = [&](float a, float b, uint32_t &hi, uint32_t &lo) {
        if constexpr (NW == 4)
            split_bf16x2(a, b, hi, lo, sk);
        else
            split_bf16x2(a, b, hi, lo);
    };

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
            if (OUTS == 0 || OUTS == 2)  // state maps read neither Q nor P'
                return;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(cs.q, (GDN_LDS void *)&B.Q[64 * (win - 16)], 16, woff[i], 0, 0, 0);
        } else if (NW * i < 32 + VWIN) {
            if (OUTS == 2)  // identity rows: V = 0
                return;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(cs.v, (GDN_LDS void *)&B.V[64 * (win - 32)], 16, woff[i], 0, 0, 0);
        } else if (win < NWIN) {
            const int r = win - 32 - VWIN;
            if (r < 18) {
                const int mt = r / 6, pr = r % 6, b = pr == 0 ? 0 : (pr == 1 ? 2 : pr + 2);
                if ((OUTS == 0 || OUTS == 2) && mt == 2)
                    return;
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
                split2(S[2 * ks][0], S[2 * ks][1], h0, l0);
                split2(S[2 * ks][2], S[2 * ks][3], h1, l1);
                split2(S[2 * ks + 1][0], S[2 * ks + 1][1], h2, l2);
                split2(S[2 * ks + 1][2], S[2 * ks + 1][3], h3, l3);
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
    // A chunk is two halves: phase1 = (a) X = K S0^T, (b) R = V - gamma X, (c) U = T' R;
    // phase2 = (d) W = dec U, (e) the outputs, (f) the state update. The next chunk's
    // copies (PER windows per wave) are spread over phase1: issued all at once they queue
    // behind each other and stall the issuing waves.
    u32x4 Bh[4];  // S0 hi, from phase1 (a) to phase2 (e)
    f32x4 U[4];   // phase1 (c) -> phase2 (d)
    f32x4 dc[4];  // the gate area's dec, read in phase1 (c) for phase2 (d)
    auto issue_slot = [&](ScanBuf<NW> &Bn, const ChunkSrc &ncs, bool issue, const int slot) {
#pragma unroll
        for (int i = 0; i < PER; ++i)  // slots 0..7
            if ((i * 8) / PER == slot && issue)
                issue_win(Bn, ncs, i);
    };
    // copies at slots 0..7: after (a) steps 0..3 and (c) tiles 0..3
    auto phase1 = [&](ScanBuf<NW> &B, ScanBuf<NW> &Bn, const ChunkSrc &ncs, bool issue) {
        const char *Kb = (const char *)B.K, *Vb = (const char *)B.V;
        const char *Th = (const char *)B.T[0], *Tl = (const char *)B.T[1];
        const char *Gb = (const char *)B.G;
        auto kA = [&](int s, int tt) {
            return *(const u32x4 *)(Kb + koffA[s] + 256 * (32 * (tt >> 1) + 4 * (tt & 1)));
        };
        // NW == 4: S0's only other reader is (f), as gammaC S0. Scaled here (the asm keeps
        // the product from being sunk into (f)), S0 dies in the split, whose dot-product
        // residuals are then formed in S0's registers.
        const float gC4 = NW == 4 ? *(const float *)(Gb + 768) : 0.f;
        auto split_s = [&](int s, u32x4 &bh, u32x4 &bl) {
            const f32x4 s0 = S[2 * s], s1 = S[2 * s + 1];
            if constexpr (NW == 4) {
                S[2 * s] = gC4 * s0;
                S[2 * s + 1] = gC4 * s1;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    asm volatile("" : "+v"(S[2 * s][i]), "+v"(S[2 * s + 1][i]));
            }
            uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
            split2(s0[0], s0[1], h0, l0);
            split2(s0[2], s0[3], h1, l1);
            split2(s1[0], s1[1], h2, l2);
            split2(s1[2], s1[3], h3, l3);
            bh = u32x4{h0, h1, h2, h3};
            bl = u32x4{l0, l1, l2, l3};
        };

        // (a) S0 as MFMA operands (hi + lo), X = K S0^T
        u32x4 Bl[4], ka[2][4];
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
            issue_slot(Bn, ncs, issue, s);
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
            split2(r0, r1, h01, l01);
            split2(r2, r3, h23, l23);
            const int e = 2 * (tt & 1);
            Rh[tt >> 1][e] = h01; Rh[tt >> 1][e + 1] = h23;
            Rl[tt >> 1][e] = l01; Rl[tt >> 1][e + 1] = l23;
        }

        // (c) U = T' R
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
            issue_slot(Bn, ncs, issue, 4 + tt);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    auto phase2 = [&](ScanBuf<NW> &B, int c) {
        const int lenc = min(kC, len - c * kC);
        const char *Kb = (const char *)B.K, *Qb = (const char *)B.Q;
        const char *Pb = (const char *)B.P, *Gb = (const char *)B.G;

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
            split2(dc[tt][0] * U[tt][0], dc[tt][1] * U[tt][1], h01, l01);
            split2(dc[tt][2] * U[tt][2], dc[tt][3] * U[tt][3], h23, l23);
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
        // one store per output tile: the chunk barrier leaves exactly these four in flight
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
            f32x4 acc = NW == 4 ? S[gidx] : gC * S[gidx];  // NW == 4: gammaC S0 from (a)
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

    auto compute = [&](ScanBuf<NW> &B, int c, ScanBuf<NW> &Bn, bool more) {
        const ChunkSrc ncs = chunk_src(more ? c + 1 : c);
        phase1(B, Bn, ncs, more);
        phase2(B, c);
    };
    // The barrier before a chunk waits for this wave's copies of it (vector memory
    // operations complete in issue order). After the first chunk, a job with outputs
    // has issued exactly four more operations since those copies: the previous chunk's
    // output stores, which nothing in the kernel reads, so it leaves them in flight
    // (waiting for them cost ~700 of a chunk's ~7000 cycles). Before the first chunk,
    // state loads the compiler may have ordered either way are in flight: wait for all.
    const bool keep_stores = do_out;
    auto chunk_barrier = [&](bool first) {
        if (keep_stores && !first) {
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_waitcnt(0x0074);  // vmcnt(4) lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        } else {
            dma_barrier();
        }
    };
    for (int c = cb; c < ce; c += 2) {
        chunk_barrier(c == cb);  // chunk c is in BA; every wave is done with BB
        compute(BA, c, BB, c + 1 < ce);
        if (c + 1 >= ce)
            break;
        chunk_barrier(false);
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
            split2(a[0], a[1], h0, l0);
            split2(a[2], a[3], h1, l1);
            split2(b[0], b[1], h2, l2);
            split2(b[2], b[3], h3, l3);
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

// The kernel's argument block through a pointer taken from the kernarg segment register and
// passed through an empty asm, so the compiler cannot prove it equal to the one behind the
// kernel parameter or another call's. A body given it keeps its own argument loads: with
// several bodies in one kernel on one pointer, the compiler merged their loads of the same
// fields above the branch and kept them live through every loop (scan4 segment kernel with
// two bodies: 102 SGPRs spilled instead of 26; the segment passes ran up to 3 % slower).
__device__ __forceinline__ const ScanArgs &fresh_kernel_args()
{
    typedef const ScanArgs __attribute__((address_space(4))) *KArgs;
    KArgs kp = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kp));
    return *(const ScanArgs *)kp;
}

// A segment kernel holds four bodies, each on its own argument pointer: a whole sequence
// listed in the job table (kJobFirst without a slot: from the initial state, outputs, final
// state into new_state) takes the whole-sequence body, whose loop carries none of the segment
// code; segment jobs with outputs and the two kinds of state map take one body each.
// Measured on MI355X, bit-identical against one segment body for every job: the qk4_v8
// prefills of 8 sequences (all whole, or mixed with cut ones) 44.4 -> 40.9 and 54.9 -> 49.9
// us; 1 x 4096 at 32 v-heads 98.4 -> 91.9 us.
template <int NW, bool SEG>
__device__ __forceinline__ void scan_kernel_body(const ScanArgs &p, ScanBuf<NW> &BA,
                                                 ScanBuf<NW> &BB)
{
    ScanJob job;
    if (!scan_job<NW, SEG>(p, job))
        return;
    if constexpr (SEG) {
        if (job.kind == kJobFirst && job.q < 0 && job.cb == 0) {
            scan_body<NW, false, 1>(fresh_kernel_args(), job, BA, BB);
        } else if (job.kind == kJobFirst || job.kind == kJobResume) {
            scan_body<NW, true, 0, 1>(fresh_kernel_args(), job, BA, BB);
        } else if (job.kind == kJobZero) {
            scan_body<NW, true, 0, 0>(fresh_kernel_args(), job, BA, BB);
        } else {
            scan_body<NW, true, 0, 2>(fresh_kernel_args(), job, BA, BB);
        }
    } else {
        scan_body<NW, SEG>(p, job, BA, BB);
    }
}

template <bool SEG>
__global__ __launch_bounds__(512) void gdn_prefill_scan8_kernel(ScanArgs p)
{
    __shared__ ScanBuf<8> bufA, bufB;
    scan_kernel_body<8, SEG>(p, bufA, bufB);
}

template <bool SEG>
__global__ __launch_bounds__(256) void gdn_prefill_scan4_kernel(ScanArgs p)
{
    __shared__ ScanBuf<4> bufA, bufB;
    scan_kernel_body<4, SEG>(p, bufA, bufB);
}

template __global__ void gdn_prefill_scan8_kernel<false>(ScanArgs p);
template __global__ void gdn_prefill_scan8_kernel<true>(ScanArgs p);
template __global__ void gdn_prefill_scan4_kernel<false>(ScanArgs p);
template __global__ void gdn_prefill_scan4_kernel<true>(ScanArgs p);

}  // namespace gdn
