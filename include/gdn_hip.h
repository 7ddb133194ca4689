/*
 * gdn_hip.h -- C ABI of the MI355X (gfx950) Gated DeltaNet kernels.
 *
 * Plain C: raw device pointers, element strides and sizes; no torch types.
 * Every entry point returns 0 on success or a negative GDN_E* code, in which
 * case gdn_last_error() describes the failure (per calling thread; each call clears
 * it first). A HIP error that an earlier call left pending on the thread is drained
 * before the launches, so that it is not blamed on this call, and named in
 * gdn_last_error() (starting "note:") even when the call succeeds. Argument errors
 * are reported before anything is launched; after GDN_ELAUNCH, kernels launched
 * before the failing one may already have written part of the outputs. Launches are
 * asynchronous on the given stream (a hipStream_t; NULL = the default stream);
 * nothing here allocates, frees or synchronises caller memory.
 *
 * Reference interfaces these replace (codeblossom99/MLSys26-Flashinfer-AI-Kernel-
 * Generation-Contest):
 *   gdn_decode_launch   <- the Triton launch gdn_decode_kernel[grid](...) at
 *                          gdn_decode/solution/triton/kernel.py:249-270 (kernel :71-218)
 *   gdn_prefill_launch  <- the Triton launch gdn_prefill_chunk_kernel[grid](...) at
 *                          gdn_prefill/solution/triton/kernel.py:312-335 (kernel :28-250)
 *   The contest's native-binding slot for both is the TVM-FFI function
 *   "flashinfer.kernel" (gdn_decode/solution/cuda/binding.py:14-25,
 *   gdn_prefill/solution/cuda/binding.py:14-25), an empty template there.
 */
#ifndef GDN_HIP_H
#define GDN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_HIP_ABI_VERSION 1

/* Status codes. */
#define GDN_OK 0
#define GDN_EINVAL -1     /* bad sizes, null pointers, struct_size mismatch   */
#define GDN_ELAYOUT -2    /* stride / alignment the kernels do not accept      */
#define GDN_EWORKSPACE -3 /* prefill workspace missing or too small            */
#define GDN_ELAUNCH -4    /* HIP reported an error at launch                   */

/* Version of this ABI (GDN_HIP_ABI_VERSION of the build). */
int gdn_abi_version(void);

/* Message of this thread's last call ("" if it succeeded). */
const char *gdn_last_error(void);

/*
 * Single-token decode (gdn_decode/solution/triton/kernel.py:221-272).
 * Tensor layouts (strides in elements, innermost dimension must have stride 1):
 *   q, k       bf16 [B, T, HQK, D]       v, output  bf16 [B, T, HV, D]
 *   state      f32  [B, HV, D, D] (k-last: [.., v, k]); NULL = zero initial state
 *   new_state  f32  [B, HV, D, D]; may alias state exactly (in-place update)
 *   A_log, dt_bias  f32 [HV]            a, b       bf16 [B, T, HV]
 * Constraints: T >= 1, D == 128, HV % HQK == 0; state / new_state 16-byte aligned
 * with v/h/b strides multiples of 4; q/k/v/output 8-byte aligned with outer strides
 * multiples of 4.
 * T > 1: every token is one step from the input state, as each per-token program of
 * gdn_decode/solution/triton/kernel.py:110-118,146-147 loads it; new_state receives
 * the last token's update, and must not alias state (GDN_EINVAL).
 */
typedef struct gdn_decode_params {
    int32_t struct_size; /* = sizeof(gdn_decode_params) */
    int32_t batch;       /* B */
    int32_t seq_len;     /* T (1 in the reference's workloads) */
    int32_t num_qk_heads;
    int32_t num_v_heads; /* a multiple of num_qk_heads, at most 65535 */
    int32_t head_size;   /* D */
    float scale;         /* readout scale; the caller resolves 0 -> 1/sqrt(D) */
    int32_t variant;     /* must be 0 (the tuned kernel); anything else: GDN_EINVAL */
    const void *q;        int64_t q_stride[4];
    const void *k;        int64_t k_stride[4];
    const void *v;        int64_t v_stride[4];
    const float *state;   int64_t state_stride[4];
    const float *A_log;   int64_t A_log_stride;
    const void *a;        int64_t a_stride[3];
    const float *dt_bias; int64_t dt_bias_stride;
    const void *b;        int64_t b_stride[3];
    void *output;         int64_t output_stride[4];
    float *new_state;     int64_t new_state_stride[4];
} gdn_decode_params;

int gdn_decode_launch(const gdn_decode_params *p, void *stream);

/*
 * Packed variable-length prefill (gdn_prefill/solution/triton/kernel.py:253-337).
 * Tensor layouts (strides in elements, innermost dimension stride 1):
 *   q, k       bf16 [T, HQK, D]          v, output  bf16 [T, HV, D]
 *   a, b       bf16 [T, HV]              A_log, dt_bias f32 [HV]
 *   cu_seqlens int32 or int64 [N + 1], non-decreasing, cu[N] <= T (device memory)
 *   state      f32  [N, HV, D, D]; NULL = zero initial state
 *   new_state  f32  [N, HV, D, D]; may alias state exactly
 * Every output row of a token outside all [cu[n], cu[n+1]) is written as zero, as
 * the reference zero-fills output (gdn_prefill/solution/triton/kernel.py:281-286).
 * workspace: device scratch of at least gdn_prefill_workspace_size(...) bytes,
 * 256-byte aligned, owned by the caller; contents need not be initialised and are
 * rewritten by every call (two calls sharing one workspace must be stream-ordered).
 */
typedef struct gdn_prefill_params {
    int32_t struct_size; /* = sizeof(gdn_prefill_params) */
    int32_t total_tokens; /* T */
    int32_t num_seqs;     /* N */
    int32_t num_qk_heads;
    int32_t num_v_heads;
    int32_t head_size;    /* D (must be 128) */
    float scale;
    int32_t cu_seqlens_int64; /* 1: int64 cu_seqlens, 0: int32 */
    int32_t variant;      /* 0 = tuned default. 1 / 2 scan every sequence whole (no
                             segments) with 4 / 8 scan waves per workgroup;
                             anything else: GDN_EINVAL */
    int32_t reserved;     /* 0 */
    const void *q;        int64_t q_stride[3];
    const void *k;        int64_t k_stride[3];
    const void *v;        int64_t v_stride[3];
    const float *state;   int64_t state_stride[4];
    const float *A_log;   int64_t A_log_stride;
    const void *a;        int64_t a_stride[2];
    const float *dt_bias; int64_t dt_bias_stride;
    const void *b;        int64_t b_stride[2];
    const void *cu_seqlens;
    void *output;         int64_t output_stride[3];
    float *new_state;     int64_t new_state_stride[4];
    void *workspace;
    int64_t workspace_bytes;
} gdn_prefill_params;

/* Bytes of workspace gdn_prefill_launch needs for these sizes (< 0 on bad sizes). */
int64_t gdn_prefill_workspace_size(int32_t total_tokens, int32_t num_seqs,
                                   int32_t num_qk_heads, int32_t num_v_heads,
                                   int32_t head_size);

int gdn_prefill_launch(const gdn_prefill_params *p, void *stream);

/*
 * gdn_prefill_launch without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference, which keeps its prefill state in registers.
 * The workspace is a static device array of gdn_prefill_noalloc_capacity() bytes
 * (96 MiB) per device, set up on the first call on that device and held until the
 * process ends; p->workspace and p->workspace_bytes are ignored. Sizes whose
 * gdn_prefill_workspace_size exceeds it fail with GDN_EWORKSPACE before any launch
 * (at 32 v-heads: about 11,000 tokens in 16 sequences). Calls on one device share the
 * array: calls that overlap in time on one device (other streams, unordered host
 * threads) race. Nothing is allocated, freed or memset.
 */
int64_t gdn_prefill_noalloc_capacity(void);
int gdn_prefill_launch_noalloc(const gdn_prefill_params *p, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_HIP_H */
