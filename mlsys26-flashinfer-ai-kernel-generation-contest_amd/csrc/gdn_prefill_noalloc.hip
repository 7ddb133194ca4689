// Prefill entry point that allocates nothing: gdn_prefill_launch with its workspace in a
// file-scope device array instead of a caller-provided buffer, for callers that cannot
// allocate (code under HIP graph capture, tight serving loops, harnesses that forbid it).
//
// The array lives in this translation unit's own code object. The runtime loads a code
// object and allocates its globals on a device when one of its symbols is first used there
// (deferred loading, the HIP runtime's default), so a process holds the array on a device
// only once it calls this entry point there, and then until the process ends (measured on
// MI355X: a decode-only process keeps the 96 MiB free; the first call takes them). Every call on one device shares that device's array: calls that overlap
// in time on one device (different streams, or host threads without stream ordering)
// race on it. Nothing in it needs to start at zero: the plan kernel writes every table
// entry the later kernels read before they run.
#include <mutex>

#include "gdn_prefill.h"

namespace {

constexpr int64_t kScratchBytes = int64_t(96) << 20;  // 96 MiB per device
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_mu;
void *g_scratch[kMaxDevices];  // device address of `scratch` on each device (null: unresolved)

// Device address of `scratch` on device dev, resolved once per device with that device
// current. Host code never uses the array's name as an address: on the host it is a
// stand-in symbol, not device memory. Resolving it may load this code object and allocate
// its globals, which a stream capture must not record: while `st` is being captured an
// unresolved device is an error (the first call on a device comes before any capture).
int scratch_ptr(int dev, hipStream_t st, void **out)
{
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
            return gdn_set_error(GDN_EINVAL, "gdn_prefill_launch_noalloc: the first call on "
                                 "device %d is inside a stream capture; make one call on "
                                 "that device before capturing (it resolves the static "
                                 "scratch)", dev);
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess)
            return gdn_set_error(GDN_ELAUNCH, "gdn_prefill_launch_noalloc: hipGetDevice failed");
        if (cur != dev && hipSetDevice(dev) != hipSuccess)
            return gdn_set_error(GDN_ELAUNCH, "gdn_prefill_launch_noalloc: hipSetDevice(%d) failed", dev);
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev)
            (void)hipSetDevice(cur);
        if (e != hipSuccess || !p)
            return gdn_set_error(GDN_ELAUNCH, "gdn_prefill_launch_noalloc: hipGetSymbolAddress "
                                 "on device %d: %s", dev, hipGetErrorString(e));
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return GDN_OK;
}

}  // namespace

extern "C" int64_t gdn_prefill_noalloc_capacity(void) { return kScratchBytes; }

extern "C" int gdn_prefill_launch_noalloc(const gdn_prefill_params *p, void *stream)
{
    gdn_begin_call();
    if (!p || p->struct_size != (int32_t)sizeof(gdn_prefill_params))
        return gdn_set_error(GDN_EINVAL, "gdn_prefill_launch_noalloc: params NULL or struct_size mismatch");
    const int64_t need = gdn_prefill_workspace_size(p->total_tokens, p->num_seqs, p->num_qk_heads,
                                                    p->num_v_heads, p->head_size);
    if (need < 0)
        return (int)need;  // message set by gdn_prefill_workspace_size
    if (need > kScratchBytes)
        return gdn_set_error(GDN_EWORKSPACE,
                             "gdn_prefill_launch_noalloc: T=%d N=%d HV=%d needs %lld bytes of "
                             "workspace, above the %lld-byte static scratch; call "
                             "gdn_prefill_launch with a caller-owned workspace instead",
                             p->total_tokens, p->num_seqs, p->num_v_heads, (long long)need,
                             (long long)kScratchBytes);
    int dev = -1;
    hipStream_t st = (hipStream_t)stream;
    if (st == nullptr || hipStreamGetDevice(st, &dev) != hipSuccess)
        if (hipGetDevice(&dev) != hipSuccess)
            return gdn_set_error(GDN_ELAUNCH, "gdn_prefill_launch_noalloc: no current device");
    if (dev < 0 || dev >= kMaxDevices)
        return gdn_set_error(GDN_EINVAL, "gdn_prefill_launch_noalloc: device %d out of range", dev);
    void *ws = nullptr;
    const int rc = scratch_ptr(dev, st, &ws);
    if (rc)
        return rc;
    gdn_prefill_params q = *p;
    q.workspace = ws;
    q.workspace_bytes = kScratchBytes;
    return gdn_prefill_launch(&q, stream);
}
