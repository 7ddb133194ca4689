// A native C++ caller of the C ABI (include/gdn_hip.h): no Python and no torch in the
// process. It fills gdn_decode_params / gdn_prefill_params the way a C or C++ host
// would, on buffers from hipMalloc and a stream of its own, and checks the results
// against the float64 CPU oracle (oracle/liboracle_gdn.so, test infrastructure).
//
// Cases: decode (separate and in-place new_state), prefill over packed sequences with
// an empty sequence and uncovered trailing tokens (int64 cu_seqlens), and the error
// paths (struct_size mismatch, unsupported head size, workspace too small).
//
// Exit status: 0 all cases pass, 1 a case failed, 77 no HIP device (the CPU tests run
// the program only to show that it loads and links).
#include <hip/hip_runtime.h>

#include "gdn_hip.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

extern "C" int oracle_decode_f64(int B, int HQK, int HV, int D, const uint16_t *q,
                                 const uint16_t *k, const uint16_t *v, const float *state,
                                 const float *A_log, const uint16_t *a, const float *dt_bias,
                                 const uint16_t *b, double scale, double *out,
                                 double *new_state, int nthreads);
extern "C" int oracle_prefill_f64(int T, int N, int HQK, int HV, int D, const uint16_t *q,
                                  const uint16_t *k, const uint16_t *v, const float *state,
                                  const float *A_log, const uint16_t *a,
                                  const float *dt_bias, const uint16_t *b,
                                  const int64_t *cu_seqlens, double scale, double *out,
                                  double *new_state, int nthreads);

namespace {

constexpr int D = 128;
int g_failures = 0;

#define HIP_OK(x)                                                                         \
    do {                                                                                  \
        hipError_t e_ = (x);                                                              \
        if (e_ != hipSuccess) {                                                           \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);    \
            std::exit(1);                                                                 \
        }                                                                                 \
    } while (0)

// Deterministic inputs: xorshift64* uniform in [0, 1).
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
    double uniform()
    {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return (double)((s * 0x2545F4914F6CDD1Dull) >> 11) * (1.0 / 9007199254740992.0);
    }
    float sym(float r) { return (float)((2.0 * uniform() - 1.0) * r); }
};

// float -> bf16 bits, round to nearest even (finite inputs)
uint16_t bf16(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float from_bf16(uint16_t h)
{
    const uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// rows of D values, each scaled to unit L2 norm (q and k are normalised per head)
std::vector<uint16_t> unit_rows(Rng &r, size_t rows)
{
    std::vector<uint16_t> out(rows * D);
    std::vector<float> x(D);
    for (size_t i = 0; i < rows; ++i) {
        double n2 = 0;
        for (int d = 0; d < D; ++d) {
            x[d] = r.sym(1.f);
            n2 += (double)x[d] * x[d];
        }
        const float inv = (float)(1.0 / std::sqrt(n2));
        for (int d = 0; d < D; ++d)
            out[i * D + d] = bf16(x[d] * inv);
    }
    return out;
}

std::vector<uint16_t> bf16_values(Rng &r, size_t n, float range)
{
    std::vector<uint16_t> out(n);
    for (auto &x : out)
        x = bf16(r.sym(range));
    return out;
}

template <typename T>
T *to_device(const std::vector<T> &h)
{
    T *d = nullptr;
    HIP_OK(hipMalloc(&d, h.size() * sizeof(T)));
    HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <typename T>
std::vector<T> to_host(const T *d, size_t n)
{
    std::vector<T> h(n);
    HIP_OK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

// The parity rule of the tests: outputs fail an element only past both atol = rtol = 1e-2;
// new_state past both atol 1e-4 / rtol 1e-3, and normwise within 1e-3.
void check(const char *name, const std::vector<uint16_t> &out, const std::vector<double> &ref_out,
           const std::vector<float> &ns, const std::vector<double> &ref_ns)
{
    size_t out_fail = 0, ns_fail = 0;
    double out_max = 0, d2 = 0, r2 = 0;
    for (size_t i = 0; i < out.size(); ++i) {
        const double d = std::fabs((double)from_bf16(out[i]) - ref_out[i]);
        out_max = d > out_max ? d : out_max;
        out_fail += (d > 1e-2 && d > 1e-2 * std::fabs(ref_out[i])) || !std::isfinite(d);
    }
    for (size_t i = 0; i < ns.size(); ++i) {
        const double d = std::fabs((double)ns[i] - ref_ns[i]);
        ns_fail += (d > 1e-4 && d > 1e-3 * std::fabs(ref_ns[i])) || !std::isfinite(d);
        d2 += d * d;
        r2 += ref_ns[i] * ref_ns[i];
    }
    const double norm_rel = r2 > 0 ? std::sqrt(d2 / r2) : std::sqrt(d2);
    const bool ok = out_fail == 0 && ns_fail == 0 && norm_rel <= 1e-3;
    std::printf("%-34s %s  output max abs err %.3e (%zu failing)  new_state norm rel err %.3e "
                "(%zu failing)\n", name, ok ? "PASSED" : "FAILED", out_max, out_fail, norm_rel,
                ns_fail);
    g_failures += !ok;
}

void expect_code(const char *name, int rc, int want)
{
    const char *msg = gdn_last_error();
    const bool ok = rc == want && msg && msg[0] != '\0';
    std::printf("%-34s %s  code %d (want %d): %s\n", name, ok ? "PASSED" : "FAILED", rc, want,
                msg ? msg : "(null)");
    g_failures += !ok;
}

void contiguous(int64_t *st, const int64_t *shape, int n)
{
    st[n - 1] = 1;
    for (int i = n - 2; i >= 0; --i)
        st[i] = st[i + 1] * shape[i + 1];
}

void decode_case(hipStream_t stream, bool in_place)
{
    const int B = 3, HQK = 2, HV = 4;
    Rng r(in_place ? 11 : 7);
    auto q = unit_rows(r, (size_t)B * HQK), k = unit_rows(r, (size_t)B * HQK);
    auto v = bf16_values(r, (size_t)B * HV * D, 1.f);
    auto a = bf16_values(r, (size_t)B * HV, 2.f), b = bf16_values(r, (size_t)B * HV, 2.f);
    std::vector<float> A_log(HV), dt_bias(HV), state((size_t)B * HV * D * D);
    for (int h = 0; h < HV; ++h) {
        A_log[h] = (float)(r.uniform() * std::log(16.0));
        dt_bias[h] = r.sym(1.f);
    }
    for (auto &x : state)
        x = r.sym(0.05f);
    const double scale = 1.0 / std::sqrt((double)D);

    std::vector<double> ref_out((size_t)B * HV * D), ref_ns(state.size());
    oracle_decode_f64(B, HQK, HV, D, q.data(), k.data(), v.data(), state.data(), A_log.data(),
                      a.data(), dt_bias.data(), b.data(), scale, ref_out.data(), ref_ns.data(), 4);

    uint16_t *dq = to_device(q), *dk = to_device(k), *dv = to_device(v), *da = to_device(a),
             *db = to_device(b);
    float *dA = to_device(A_log), *ddt = to_device(dt_bias), *dst = to_device(state);
    uint16_t *dout = nullptr;
    HIP_OK(hipMalloc(&dout, ref_out.size() * 2));
    float *dns = dst;
    if (!in_place)
        HIP_OK(hipMalloc(&dns, state.size() * 4));

    gdn_decode_params p;
    std::memset(&p, 0, sizeof(p));
    p.struct_size = (int32_t)sizeof(p);
    p.batch = B;
    p.seq_len = 1;
    p.num_qk_heads = HQK;
    p.num_v_heads = HV;
    p.head_size = D;
    p.scale = (float)scale;
    const int64_t qs[4] = {B, 1, HQK, D}, vs[4] = {B, 1, HV, D}, ss[4] = {B, HV, D, D},
                  gs[3] = {B, 1, HV};
    p.q = dq;
    contiguous(p.q_stride, qs, 4);
    p.k = dk;
    contiguous(p.k_stride, qs, 4);
    p.v = dv;
    contiguous(p.v_stride, vs, 4);
    p.state = dst;
    contiguous(p.state_stride, ss, 4);
    p.A_log = dA;
    p.A_log_stride = 1;
    p.a = da;
    contiguous(p.a_stride, gs, 3);
    p.dt_bias = ddt;
    p.dt_bias_stride = 1;
    p.b = db;
    contiguous(p.b_stride, gs, 3);
    p.output = dout;
    contiguous(p.output_stride, vs, 4);
    p.new_state = dns;
    contiguous(p.new_state_stride, ss, 4);

    const int rc = gdn_decode_launch(&p, stream);
    if (rc != GDN_OK) {
        std::printf("gdn_decode_launch failed: %d %s\n", rc, gdn_last_error());
        std::exit(1);
    }
    HIP_OK(hipStreamSynchronize(stream));
    check(in_place ? "decode B=3 (in place)" : "decode B=3", to_host(dout, ref_out.size()),
          ref_out, to_host(dns, state.size()), ref_ns);

    if (!in_place) {
        gdn_decode_params bad = p;
        bad.struct_size = 0;
        expect_code("decode, struct_size mismatch", gdn_decode_launch(&bad, stream), GDN_EINVAL);
        bad = p;
        bad.head_size = 64;
        expect_code("decode, head size 64", gdn_decode_launch(&bad, stream), GDN_EINVAL);
        HIP_OK(hipFree(dns));
    }
    for (void *ptr : {(void *)dq, (void *)dk, (void *)dv, (void *)da, (void *)db, (void *)dA,
                      (void *)ddt, (void *)dst, (void *)dout})
        HIP_OK(hipFree(ptr));
}

void prefill_case(hipStream_t stream)
{
    const int HQK = 2, HV = 4;
    const std::vector<int64_t> cu = {0, 70, 70, 200};  // an empty sequence in the middle
    const int N = (int)cu.size() - 1, T = 205;           // tokens 200..204 belong to none
    Rng r(23);
    auto q = unit_rows(r, (size_t)T * HQK), k = unit_rows(r, (size_t)T * HQK);
    auto v = bf16_values(r, (size_t)T * HV * D, 1.f);
    auto a = bf16_values(r, (size_t)T * HV, 2.f), b = bf16_values(r, (size_t)T * HV, 2.f);
    std::vector<float> A_log(HV), dt_bias(HV), state((size_t)N * HV * D * D);
    for (int h = 0; h < HV; ++h) {
        A_log[h] = (float)(r.uniform() * std::log(4.0));
        dt_bias[h] = r.sym(1.f);
    }
    for (auto &x : state)
        x = r.sym(0.05f);
    const double scale = 1.0 / std::sqrt((double)D);

    std::vector<double> ref_out((size_t)T * HV * D), ref_ns(state.size());
    oracle_prefill_f64(T, N, HQK, HV, D, q.data(), k.data(), v.data(), state.data(),
                       A_log.data(), a.data(), dt_bias.data(), b.data(), cu.data(), scale,
                       ref_out.data(), ref_ns.data(), 4);

    uint16_t *dq = to_device(q), *dk = to_device(k), *dv = to_device(v), *da = to_device(a),
             *db = to_device(b);
    float *dA = to_device(A_log), *ddt = to_device(dt_bias), *dst = to_device(state);
    int64_t *dcu = to_device(cu);
    // the output starts as garbage: rows outside every sequence must come back as zero
    std::vector<uint16_t> junk((size_t)T * HV * D, bf16(3.f));
    uint16_t *dout = to_device(junk);
    float *dns = nullptr;
    HIP_OK(hipMalloc(&dns, state.size() * 4));

    const int64_t ws_bytes = gdn_prefill_workspace_size(T, N, HQK, HV, D);
    if (ws_bytes <= 0) {
        std::printf("gdn_prefill_workspace_size failed: %lld %s\n", (long long)ws_bytes,
                    gdn_last_error());
        std::exit(1);
    }
    void *ws = nullptr;
    HIP_OK(hipMalloc(&ws, (size_t)ws_bytes));  // hipMalloc is 256-byte aligned

    gdn_prefill_params p;
    std::memset(&p, 0, sizeof(p));
    p.struct_size = (int32_t)sizeof(p);
    p.total_tokens = T;
    p.num_seqs = N;
    p.num_qk_heads = HQK;
    p.num_v_heads = HV;
    p.head_size = D;
    p.scale = (float)scale;
    p.cu_seqlens_int64 = 1;
    const int64_t qs[3] = {T, HQK, D}, vs[3] = {T, HV, D}, ss[4] = {N, HV, D, D},
                  gs[2] = {T, HV};
    p.q = dq;
    contiguous(p.q_stride, qs, 3);
    p.k = dk;
    contiguous(p.k_stride, qs, 3);
    p.v = dv;
    contiguous(p.v_stride, vs, 3);
    p.state = dst;
    contiguous(p.state_stride, ss, 4);
    p.A_log = dA;
    p.A_log_stride = 1;
    p.a = da;
    contiguous(p.a_stride, gs, 2);
    p.dt_bias = ddt;
    p.dt_bias_stride = 1;
    p.b = db;
    contiguous(p.b_stride, gs, 2);
    p.cu_seqlens = dcu;
    p.output = dout;
    contiguous(p.output_stride, vs, 3);
    p.new_state = dns;
    contiguous(p.new_state_stride, ss, 4);
    p.workspace = ws;
    p.workspace_bytes = ws_bytes;

    const int rc = gdn_prefill_launch(&p, stream);
    if (rc != GDN_OK) {
        std::printf("gdn_prefill_launch failed: %d %s\n", rc, gdn_last_error());
        std::exit(1);
    }
    HIP_OK(hipStreamSynchronize(stream));
    check("prefill lens 70, 0, 130 + 5 gap", to_host(dout, ref_out.size()), ref_out,
          to_host(dns, state.size()), ref_ns);

    gdn_prefill_params bad = p;
    bad.workspace_bytes = ws_bytes - 256;
    expect_code("prefill, workspace too small", gdn_prefill_launch(&bad, stream),
                GDN_EWORKSPACE);

    for (void *ptr : {(void *)dq, (void *)dk, (void *)dv, (void *)da, (void *)db, (void *)dA,
                      (void *)ddt, (void *)dst, (void *)dcu, (void *)dout, (void *)dns, ws})
        HIP_OK(hipFree(ptr));
}

}  // namespace

int main()
{
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
        std::printf("no HIP device\n");
        return 77;
    }
    std::printf("gdn_abi_version %d (header %d)\n", gdn_abi_version(), GDN_HIP_ABI_VERSION);
    if (gdn_abi_version() != GDN_HIP_ABI_VERSION)
        return 1;
    HIP_OK(hipSetDevice(0));
    hipStream_t stream;
    HIP_OK(hipStreamCreate(&stream));
    decode_case(stream, false);
    decode_case(stream, true);
    prefill_case(stream);
    HIP_OK(hipStreamDestroy(stream));
    std::printf("%s\n", g_failures ? "FAILED" : "all cases PASSED");
    return g_failures ? 1 : 0;
}
