// Per-call fast path of the Python entry points: validates a destination-passing
// gdn_decode call and fills the C-ABI params in C++, then launches on torch's current
// HIP stream of the inputs' device. Python validation and ctypes marshalling cost about
// 30 us per call, ten times a small decode kernel; this path costs about 1 us.
//
// decode() returns 0 after a successful launch and 1 when the call needs the general
// Python path (default outputs to allocate, layouts the kernel cannot read or write in
// place, in-place with a token axis, a tensor scale, or anything it does not accept):
// that path then validates again and raises the reference wrapper's errors. A non-zero
// ABI code raises RuntimeError with gdn_last_error().
//
// Host-only C++ built with torch's extension builder (no device code here); the ABI
// entry points come from libgdn_hip.so as function pointers handed over by init().
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include "gdn_hip.h"

namespace {

using DecodeFn = int (*)(const gdn_decode_params *, void *);
using LastErrorFn = const char *(*)();

DecodeFn g_decode = nullptr;
LastErrorFn g_last_error = nullptr;

void init(int64_t decode_fn, int64_t last_error_fn)
{
    g_decode = reinterpret_cast<DecodeFn>(decode_fn);
    g_last_error = reinterpret_cast<LastErrorFn>(last_error_fn);
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
        throw std::runtime_error(std::string("gdn_decode_launch failed (code ") +
                                 std::to_string(rc) + "): " + (g_last_error ? g_last_error() : ""));
    return 0;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m)
{
    m.def("init", &init, "hand over the C-ABI entry points (addresses from libgdn_hip.so)");
    m.def("decode", &decode, "validate a DPS gdn_decode call and launch it; 1 = not eligible");
}
