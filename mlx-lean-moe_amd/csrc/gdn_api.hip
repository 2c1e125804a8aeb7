// C-ABI bookkeeping plus the two elementwise kernels of the path: the gates
// (forget gate and beta) and the gated RMSNorm epilogue.
#include <stdarg.h>
#include <stdio.h>

#include "gdn_common.h"
#include "gdn_host.h"

namespace gdn {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err == hipSuccess) return 0;
    fail(int(err), "%s: launch failed: %s", what, hipGetErrorString(err));
    return int(err);
}

// g = exp(-exp(A_log) * softplus(a + dt_bias)) in float32 and
// beta = sigmoid(b) in beta's dtype (gated_delta.py:14-21, linear_attention.py:116).
__global__ void gates_kernel(const void* a, const void* b, int ab_dtype, const float* A_log,
                             const float* dt_bias, float* g, void* beta, int beta_dtype,
                             int64_t n, int Hv) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int h = int(i % Hv);
    if (g) g[i] = expf(log_forget_gate(load_any(a, i, ab_dtype), A_log[h], dt_bias[h]));
    if (beta) store_any(beta, i, beta_dtype, beta_of(load_any(b, i, ab_dtype), beta_dtype));
}

// One wave per row: out = silu(z) * rms_norm(x held in out's dtype, w, eps),
// the normalised value held in out's dtype before the float product
// (linear_attention.py:22-32; the call site's y.astype(z.dtype) is the
// rounding of x to out's dtype, linear_attention.py:122-124).
__global__ void gated_rmsnorm_kernel(const void* x, int x_dtype, const void* z, int z_dtype,
                                     int64_t z_stride, int heads, const float* w, float eps,
                                     void* out, int out_dtype, int64_t rows, int D) {
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (row >= rows) return;  // uniform per wave
    const int64_t base = row * D;
    const int64_t zbase = row / heads * z_stride + row % heads * D;  // z's row of D
    float ss = 0.f;
    for (int i = lane; i < D; i += kWave) {
        const float v = round_to(load_any(x, base + i, x_dtype), out_dtype);
        ss += v * v;
    }
    ss = group_sum<kWave>(ss);
    const float r = 1.f / sqrtf(ss / float(D) + eps);
    for (int i = lane; i < D; i += kWave) {
        const float v = round_to(load_any(x, base + i, x_dtype), out_dtype);
        const float normed = round_to(v * r * w[i], out_dtype);
        const float zz = load_any(z, zbase + i, z_dtype);
        store_any(out, base + i, out_dtype, silu(zz) * normed);
    }
}

// The same for bfloat16 z and out, float32 or bfloat16 x, D = 8 kLanes and
// 16-byte aligned rows: kLanes lanes a row, 8 elements a lane, 64 / kLanes
// rows a wave.
template <int kLanes, bool kXF32>
__global__ __launch_bounds__(256) void gated_rmsnorm_vec_kernel(const void* __restrict__ x,
                                                                const uint16_t* __restrict__ z,
                                                                int64_t z_stride, int heads,
                                                                const float* __restrict__ w, float eps,
                                                                uint16_t* __restrict__ out,
                                                                int64_t rows) {
    constexpr int D = 8 * kLanes, kRows = kWave / kLanes;
    const int lane = threadIdx.x % kWave;
    const int64_t row = (int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * kRows +
                        lane / kLanes;
    const bool live = row < rows;
    const int64_t rr = live ? row : rows - 1;
    const int64_t at = rr * D + (lane % kLanes) * 8;
    const int64_t zat = rr / heads * z_stride + rr % heads * D + (lane % kLanes) * 8;
    float v[8];
    if constexpr (kXF32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + at);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + at + 4);
        const float raw[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = round_bf16(raw[e]);
    } else {
        unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + at), v);
    }
    float zz[8];
    unpack8(*reinterpret_cast<const uint4*>(z + zat), zz);
    const float4 w0 = *reinterpret_cast<const float4*>(w + (lane % kLanes) * 8);
    const float4 w1 = *reinterpret_cast<const float4*>(w + (lane % kLanes) * 8 + 4);
    const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
    ss = group_sum<kLanes>(ss);
    const float r = 1.f / sqrtf(ss / float(D) + eps);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = silu(zz[e]) * round_bf16(v[e] * r * ww[e]);
    if (live) *reinterpret_cast<uint4*>(out + at) = pack8(o);
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_abi_version(void) { return 16; }

extern "C" const char* gdn_last_error(void) { return g_last_error; }

extern "C" int gdn_gates(const void* a, const void* b, int ab_dtype, const float* A_log,
                         const float* dt_bias, float* g, void* beta, int beta_dtype,
                         int64_t rows, int Hv, void* stream) {
    GDN_REQUIRE(rows >= 0 && Hv > 0, "gdn_gates: bad sizes rows=%lld Hv=%d", (long long)rows, Hv);
    GDN_REQUIRE(valid_dtype(ab_dtype) && valid_dtype(beta_dtype), "gdn_gates: bad dtype");
    if (rows == 0) return 0;
    GDN_REQUIRE(g || beta, "gdn_gates: neither g nor beta requested");
    GDN_REQUIRE(!g || (a && A_log && dt_bias), "gdn_gates: g needs a, A_log and dt_bias");
    GDN_REQUIRE(!beta || b, "gdn_gates: beta needs b");
    const int64_t n = rows * Hv;
    const int threads = 256;
    const int64_t blocks = (n + threads - 1) / threads;
    hipLaunchKernelGGL(gates_kernel, dim3(unsigned(blocks)), dim3(threads), 0, as_stream(stream),
                       a, b, ab_dtype, A_log, dt_bias, g, beta, beta_dtype, n, Hv);
    return check_launch("gdn_gates");
}

extern "C" int gdn_gated_rmsnorm(const void* x, int x_dtype, const void* z, int z_dtype,
                                 int64_t z_stride, int heads, const float* w, float eps, void* out,
                                 int out_dtype, int64_t rows, int D, void* stream) {
    GDN_REQUIRE(rows >= 0 && D > 0, "gdn_gated_rmsnorm: bad sizes");
    GDN_REQUIRE(heads >= 1 && rows % heads == 0 && z_stride >= int64_t(heads) * D,
                "gdn_gated_rmsnorm: z layout (heads=%d, z_stride=%lld) does not fit %lld rows of %d",
                heads, (long long)z_stride, (long long)rows, D);
    GDN_REQUIRE(valid_dtype(x_dtype) && valid_dtype(z_dtype) && valid_dtype(out_dtype),
                "gdn_gated_rmsnorm: bad dtype");
    if (rows == 0) return 0;
    GDN_REQUIRE(x && z && w && out, "gdn_gated_rmsnorm: null pointer");
    const auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if ((x_dtype == GDN_F32 || x_dtype == GDN_BF16) && z_dtype == GDN_BF16 && out_dtype == GDN_BF16 &&
        (D == 64 || D == 128 || D == 256) && aligned(x) && aligned(z) && aligned(w) && aligned(out) &&
        z_stride % 8 == 0) {
        const int64_t per_block = 4 * (kWave / (D / 8));  // rows: four waves
        const dim3 grid(static_cast<unsigned>((rows + per_block - 1) / per_block));
        const bool xf = x_dtype == GDN_F32;
        const auto* zz = static_cast<const uint16_t*>(z);
        auto* oo = static_cast<uint16_t*>(out);
        using Kernel = void (*)(const void*, const uint16_t*, int64_t, int, const float*, float, uint16_t*,
                                int64_t);
        const Kernel kern = D == 64  ? (xf ? gated_rmsnorm_vec_kernel<8, true> : gated_rmsnorm_vec_kernel<8, false>)
                          : D == 128 ? (xf ? gated_rmsnorm_vec_kernel<16, true> : gated_rmsnorm_vec_kernel<16, false>)
                                     : (xf ? gated_rmsnorm_vec_kernel<32, true> : gated_rmsnorm_vec_kernel<32, false>);
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, as_stream(stream), x, zz, z_stride, heads, w, eps, oo,
                           rows);
        return check_launch("gdn_gated_rmsnorm");
    }
    const int waves = 4;
    const int64_t blocks = (rows + waves - 1) / waves;
    hipLaunchKernelGGL(gated_rmsnorm_kernel, dim3(unsigned(blocks)), dim3(waves * kWave), 0,
                       as_stream(stream), x, x_dtype, z, z_dtype, z_stride, heads, w, eps, out, out_dtype,
                       rows, D);
    return check_launch("gdn_gated_rmsnorm");
}
