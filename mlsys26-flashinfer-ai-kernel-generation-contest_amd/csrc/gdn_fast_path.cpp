// Per-call fast path of the Python entry points: validates a destination-passing
// gdn_decode or gdn_prefill call and fills the C-ABI params in C++, then launches on
// torch's current HIP stream of the inputs' device. Python validation and ctypes
// marshalling cost about 30 us per call, ten times a small decode kernel; this path
// costs about 1 us.
//
// decode() / prefill() return 0 after a successful launch and 1 when the call needs the
// general Python path (default outputs to allocate, empty inputs, layouts the kernels
// cannot read or write in place, in-place with a token axis or other strides, a stream
// being captured into a graph (prefill: that path gives each graph its own workspace),
// or anything else they do not accept): that path then validates again and raises the
// reference wrapper's errors. A non-zero ABI code raises RuntimeError with
// gdn_last_error().
//
// Host-only C++ built with torch's extension builder (no device code here); the ABI
// entry points come from libgdn_hip.so as function pointers handed over by init().
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <cstring>
#include <map>
#include <mutex>

#include "gdn_hip.h"

namespace {

using DecodeFn = int (*)(const gdn_decode_params *, void *);
using PrefillFn = int (*)(const gdn_prefill_params *, void *);
using WsSizeFn = int64_t (*)(int32_t, int32_t, int32_t, int32_t, int32_t);
using LastErrorFn = const char *(*)();

DecodeFn g_decode = nullptr;
PrefillFn g_prefill = nullptr;
WsSizeFn g_ws_size = nullptr;
LastErrorFn g_last_error = nullptr;

void init(int64_t decode_fn, int64_t prefill_fn, int64_t ws_size_fn, int64_t last_error_fn)
{
    g_decode = reinterpret_cast<DecodeFn>(decode_fn);
    g_prefill = reinterpret_cast<PrefillFn>(prefill_fn);
    g_ws_size = reinterpret_cast<WsSizeFn>(ws_size_fn);
    g_last_error = reinterpret_cast<LastErrorFn>(last_error_fn);
}

[[noreturn]] void abi_failed(const char *what, int rc)
{
    throw std::runtime_error(std::string(what) + " failed (code " + std::to_string(rc) +
                             "): " + (g_last_error ? g_last_error() : ""));
}

bool aligned(const at::Tensor &t, int64_t bytes)
{
    return reinterpret_cast<uintptr_t>(t.data_ptr()) % bytes == 0;
}

// The kernels' direct-access rule (gdn_hip.api._layout_ok): unit innermost stride (or a
// size-1 innermost dimension), base alignment, outer strides multiples of `mult` where
// the dimension has more than one element.
bool layout_ok(const at::Tensor &t, int64_t align_bytes, int64_t mult)
{
    const int64_t nd = t.dim();
    if (t.stride(nd - 1) != 1 && t.size(nd - 1) != 1)
        return false;
    if (!aligned(t, align_bytes))
        return false;
    for (int64_t i = 0; i + 1 < nd; ++i)
        if (t.size(i) > 1 && t.stride(i) % mult != 0)
            return false;
    return true;
}

bool is(const at::Tensor &t, at::ScalarType st, int64_t ndim, const c10::Device &dev)
{
    return t.defined() && t.scalar_type() == st && t.dim() == ndim && t.device() == dev;
}

template <int N>
void strides(const at::Tensor &t, int64_t (&out)[N])
{
    for (int i = 0; i < N; ++i)
        out[i] = t.stride(i);
    if (t.size(N - 1) == 1)
        out[N - 1] = 1;  // a size-1 innermost dimension may report any stride
}

int64_t decode(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v,
               const c10::optional<at::Tensor> &state, const at::Tensor &A_log,
               const at::Tensor &a, const at::Tensor &dt_bias, const at::Tensor &b, double scale,
               const at::Tensor &output, const at::Tensor &new_state, int64_t variant)
{
    if (!g_decode || !q.defined() || !q.is_cuda())
        return 1;
    const c10::Device dev = q.device();
    using at::kBFloat16;
    using at::kFloat;
    if (!is(q, kBFloat16, 4, dev) || !is(k, kBFloat16, 4, dev) || !is(v, kBFloat16, 4, dev) ||
        !is(A_log, kFloat, 1, dev) || !is(a, kBFloat16, 3, dev) || !is(dt_bias, kFloat, 1, dev) ||
        !is(b, kBFloat16, 3, dev) || !is(output, kBFloat16, 4, dev) ||
        !is(new_state, kFloat, 4, dev))
        return 1;
    const int64_t B = q.size(0), T = q.size(1), HQK = q.size(2), D = q.size(3), HV = v.size(2);
    if (D != 128 || B < 1 || T < 1 || HQK < 1 || HV % HQK != 0 || HV > 65535 || B > INT32_MAX ||
        T > INT32_MAX)
        return 1;
    if (k.sizes() != q.sizes() || v.size(0) != B || v.size(1) != T || v.size(3) != D ||
        A_log.size(0) != HV || dt_bias.size(0) != HV || a.size(0) != B || a.size(1) != T ||
        a.size(2) != HV || b.sizes() != a.sizes() || output.sizes() != v.sizes() ||
        new_state.size(0) != B || new_state.size(1) != HV || new_state.size(2) != D ||
        new_state.size(3) != D)
        return 1;
    const bool has_state = state.has_value() && state->defined();
    if (has_state) {
        const at::Tensor &s = *state;
        if (!is(s, kFloat, 4, dev) || s.sizes() != new_state.sizes() || !layout_ok(s, 16, 4))
            return 1;
        if (s.data_ptr() == new_state.data_ptr() &&
            (T > 1 || s.strides() != new_state.strides()))
            return 1;  // the general path reads a copy of the state
    }
    if (!layout_ok(q, 8, 4) || !layout_ok(k, 8, 4) || !layout_ok(v, 1, 1) ||
        !layout_ok(a, 1, 1) || !layout_ok(b, 1, 1) || !layout_ok(output, 2, 1) ||
        !layout_ok(new_state, 16, 4))
        return 1;

    gdn_decode_params P;
    P.struct_size = sizeof(P);
    P.batch = (int32_t)B;
    P.seq_len = (int32_t)T;
    P.num_qk_heads = (int32_t)HQK;
    P.num_v_heads = (int32_t)HV;
    P.head_size = (int32_t)D;
    P.scale = scale == 0.0 ? (float)(1.0 / std::sqrt((double)D)) : (float)scale;
    P.variant = (int32_t)variant;
    P.q = q.data_ptr();
    strides(q, P.q_stride);
    P.k = k.data_ptr();
    strides(k, P.k_stride);
    P.v = v.data_ptr();
    strides(v, P.v_stride);
    P.state = has_state ? state->data_ptr<float>() : nullptr;
    if (has_state)
        strides(*state, P.state_stride);
    else
        for (auto &x : P.state_stride)
            x = 0;
    P.A_log = A_log.data_ptr<float>();
    P.A_log_stride = A_log.stride(0);
    P.a = a.data_ptr();
    strides(a, P.a_stride);
    P.dt_bias = dt_bias.data_ptr<float>();
    P.dt_bias_stride = dt_bias.stride(0);
    P.b = b.data_ptr();
    strides(b, P.b_stride);
    P.output = output.data_ptr();
    strides(output, P.output_stride);
    P.new_state = new_state.data_ptr<float>();
    strides(new_state, P.new_state_stride);

    hipStream_t stream = c10::hip::getCurrentHIPStream(dev.index()).stream();
    const int rc = g_decode(&P, (void *)stream);
    if (rc != GDN_OK)
        abi_failed("gdn_decode_launch", rc);
    return 0;
}

// Eager prefill workspaces, one grow-only buffer per (device, stream), rewritten by every
// call (stream order keeps calls on one stream apart). Held as torch tensors, so the
// memory comes from (and returns to) torch's caching allocator. The map is never
// destroyed: at process exit the allocator may already be gone.
std::mutex g_ws_mu;
auto *g_ws = new std::map<std::pair<int, hipStream_t>, at::Tensor>();

at::Tensor workspace(const c10::Device &dev, hipStream_t stream, int64_t nbytes)
{
    std::lock_guard<std::mutex> lock(g_ws_mu);
    at::Tensor &buf = (*g_ws)[{dev.index(), stream}];
    if (!buf.defined() || buf.numel() < nbytes)
        buf = at::empty({std::max<int64_t>(nbytes, int64_t(1) << 20)},
                        at::TensorOptions().dtype(at::kByte).device(dev));
    return buf;
}

void release_workspace()
{
    std::lock_guard<std::mutex> lock(g_ws_mu);
    g_ws->clear();
}

int64_t prefill(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v,
                const c10::optional<at::Tensor> &state, const at::Tensor &A_log,
                const at::Tensor &a, const at::Tensor &dt_bias, const at::Tensor &b,
                const at::Tensor &cu_seqlens, double scale, const at::Tensor &output,
                const at::Tensor &new_state, int64_t variant)
{
    if (!g_prefill || !g_ws_size || !q.defined() || !q.is_cuda())
        return 1;
    const c10::Device dev = q.device();
    using at::kBFloat16;
    using at::kFloat;
    if (!is(q, kBFloat16, 3, dev) || !is(k, kBFloat16, 3, dev) || !is(v, kBFloat16, 3, dev) ||
        !is(A_log, kFloat, 1, dev) || !is(a, kBFloat16, 2, dev) || !is(dt_bias, kFloat, 1, dev) ||
        !is(b, kBFloat16, 2, dev) || !is(output, kBFloat16, 3, dev) ||
        !is(new_state, kFloat, 4, dev) || !cu_seqlens.defined() || cu_seqlens.dim() != 1 ||
        cu_seqlens.device() != dev ||
        (cu_seqlens.scalar_type() != at::kInt && cu_seqlens.scalar_type() != at::kLong))
        return 1;
    const int64_t T = q.size(0), HQK = q.size(1), D = q.size(2), HV = v.size(1);
    const int64_t N = cu_seqlens.size(0) - 1;
    if (D != 128 || T < 1 || N < 1 || HQK < 1 || HV % HQK != 0 || T > INT32_MAX || N > INT32_MAX)
        return 1;
    if (k.sizes() != q.sizes() || v.size(0) != T || v.size(2) != D || A_log.size(0) != HV ||
        dt_bias.size(0) != HV || a.size(0) != T || a.size(1) != HV || b.sizes() != a.sizes() ||
        output.size(0) != T || output.size(1) != HV || output.size(2) != D ||
        new_state.size(0) != N || new_state.size(1) != HV || new_state.size(2) != D ||
        new_state.size(3) != D || cu_seqlens.stride(0) != 1)
        return 1;
    const bool has_state = state.has_value() && state->defined();
    if (has_state) {
        const at::Tensor &s = *state;
        if (!is(s, kFloat, 4, dev) || s.sizes() != new_state.sizes() || !layout_ok(s, 16, 4))
            return 1;
        if (s.data_ptr() == new_state.data_ptr() && s.strides() != new_state.strides())
            return 1;  // the general path reads a copy of the state
    }
    if (!layout_ok(q, 16, 8) || !layout_ok(k, 16, 8) || !layout_ok(v, 16, 8) ||
        !layout_ok(a, 1, 1) || !layout_ok(b, 1, 1) || !layout_ok(output, 16, 8) ||
        !layout_ok(new_state, 16, 4))
        return 1;
    hipStream_t stream = c10::hip::getCurrentHIPStream(dev.index()).stream();
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
        return 1;  // graphs get workspaces of their own from the general path
    const int64_t ws_bytes = g_ws_size((int32_t)T, (int32_t)N, (int32_t)HQK, (int32_t)HV,
                                       (int32_t)D);
    if (ws_bytes < 0)
        abi_failed("gdn_prefill_workspace_size", (int)ws_bytes);
    const at::Tensor ws = workspace(dev, stream, ws_bytes);

    gdn_prefill_params P;
    std::memset(&P, 0, sizeof(P));
    P.struct_size = sizeof(P);
    P.total_tokens = (int32_t)T;
    P.num_seqs = (int32_t)N;
    P.num_qk_heads = (int32_t)HQK;
    P.num_v_heads = (int32_t)HV;
    P.head_size = (int32_t)D;
    P.scale = scale == 0.0 ? (float)(1.0 / std::sqrt((double)D)) : (float)scale;
    P.cu_seqlens_int64 = cu_seqlens.scalar_type() == at::kLong ? 1 : 0;
    P.variant = (int32_t)variant;
    P.q = q.data_ptr();
    strides(q, P.q_stride);
    P.k = k.data_ptr();
    strides(k, P.k_stride);
    P.v = v.data_ptr();
    strides(v, P.v_stride);
    P.state = has_state ? state->data_ptr<float>() : nullptr;
    if (has_state)
        strides(*state, P.state_stride);
    P.A_log = A_log.data_ptr<float>();
    P.A_log_stride = A_log.stride(0);
    P.a = a.data_ptr();
    strides(a, P.a_stride);
    P.dt_bias = dt_bias.data_ptr<float>();
    P.dt_bias_stride = dt_bias.stride(0);
    P.b = b.data_ptr();
    strides(b, P.b_stride);
    P.cu_seqlens = cu_seqlens.data_ptr();
    P.output = output.data_ptr();
    strides(output, P.output_stride);
    P.new_state = new_state.data_ptr<float>();
    strides(new_state, P.new_state_stride);
    P.workspace = ws.data_ptr();
    P.workspace_bytes = ws.numel();
    const int rc = g_prefill(&P, (void *)stream);
    if (rc != GDN_OK)
        abi_failed("gdn_prefill_launch", rc);
    return 0;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m)
{
    m.def("init", &init, "hand over the C-ABI entry points (addresses from libgdn_hip.so)");
    m.def("decode", &decode, "validate a DPS gdn_decode call and launch it; 1 = not eligible");
    m.def("prefill", &prefill, "validate a DPS gdn_prefill call and launch it; 1 = not eligible");
    m.def("release_workspace", &release_workspace, "drop the cached eager prefill workspaces");
}
