// Sequential gated-delta scans over token runs.
//
// scan_reference_kernel: one thread per state row, the reference's exact
// operation order (gated_delta.py:35-39), any Dk/Dv and dtype mix. A test aid
// and the use_kernel=False path.
//
// scan_kernel: the state tile stays in registers across the token loop.
// 32 lanes own one state row (Dk/32 contiguous values each), 8 rows per
// 256-thread workgroup. Per token the lanes form S.k, S.q and k.q in one
// pass over the (undecayed) row and one 32-lane reduction, then
//     delta = beta (v - g S.k),  y = g S.q + delta (k.q),  S <- g S + delta k^T
// which is the reference's step (decay, read, delta, update, output)
// rearranged so that a token needs one reduction instead of two.
#include "gdn_common.h"
#include "gdn_host.h"

namespace gdn {

__global__ void scan_reference_kernel(const void* q, const void* k, int qk_dtype, const void* v,
                                      int v_dtype, const void* g, int g_dtype, const void* beta,
                                      int beta_dtype, const void* state_in, void* state_out,
                                      int state_dtype, void* y, int y_dtype, const int32_t* cu,
                                      int N, int64_t L_uniform, int Hk, int Hv, int Dk, int Dv) {
    const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= int64_t(N) * Hv * Dv) return;
    const int run = int(gid / (int64_t(Hv) * Dv));
    const int h = int((gid / Dv) % Hv);
    const int dv = int(gid % Dv);
    const int hk = h / (Hv / Hk);
    float S[256];
    const int64_t sbase = ((int64_t(run) * Hv + h) * Dv + dv) * Dk;
    for (int j = 0; j < Dk; ++j) S[j] = load_any(state_in, sbase + j, state_dtype);
    const int64_t t0 = cu ? cu[run] : run * L_uniform;
    const int64_t t1 = cu ? cu[run + 1] : t0 + L_uniform;
    for (int64_t t = t0; t < t1; ++t) {
        const int64_t kb = (t * Hk + hk) * Dk;
        const float gt = load_any(g, t * Hv + h, g_dtype);
        const float bt = load_any(beta, t * Hv + h, beta_dtype);
        float read = 0.f;
        for (int j = 0; j < Dk; ++j) S[j] *= gt;
        for (int j = 0; j < Dk; ++j) read += S[j] * load_any(k, kb + j, qk_dtype);
        const float delta = (load_any(v, (t * Hv + h) * Dv + dv, v_dtype) - read) * bt;
        float out = 0.f;
        for (int j = 0; j < Dk; ++j) S[j] += load_any(k, kb + j, qk_dtype) * delta;
        for (int j = 0; j < Dk; ++j) out += S[j] * load_any(q, kb + j, qk_dtype);
        store_any(y, (t * Hv + h) * Dv + dv, y_dtype, out);
    }
    for (int j = 0; j < Dk; ++j) store_any(state_out, sbase + j, state_dtype, S[j]);
}

constexpr int kScanThreads = 256;
constexpr int kScanRows = kScanThreads / 32;

struct TokenIn {
    float g, beta, v;
};

template <int NPL>
__global__ __launch_bounds__(kScanThreads) void scan_kernel(
    const void* __restrict__ q, const void* __restrict__ k, int qk_dtype,
    const void* __restrict__ v, int v_dtype, const void* __restrict__ g, int g_dtype,
    const void* __restrict__ beta, int beta_dtype, const void* state_in, void* state_out,
    int state_dtype, void* __restrict__ y, int y_dtype, const int32_t* __restrict__ cu, int N,
    int64_t L_uniform, int Hk, int Hv, int Dk, int Dv) {
    const int tiles = (Dv + kScanRows - 1) / kScanRows;
    const int tile = blockIdx.x % tiles;
    const int h = (blockIdx.x / tiles) % Hv;
    const int run = blockIdx.x / (tiles * Hv);
    const int l32 = threadIdx.x & 31;
    const int row = tile * kScanRows + threadIdx.x / 32;
    const bool active = row < Dv;
    const int hk = h / (Hv / Hk);
    const int col = l32 * NPL;

    float S[NPL];
    const int64_t sbase = ((int64_t(run) * Hv + h) * Dv + row) * Dk + col;
#pragma unroll
    for (int j = 0; j < NPL; ++j) S[j] = active ? load_any(state_in, sbase + j, state_dtype) : 0.f;

    const int64_t t0 = cu ? cu[run] : run * L_uniform;
    const int64_t t1 = cu ? cu[run + 1] : t0 + L_uniform;

    // Token t+1's inputs are fetched while token t is processed.
    float kn[NPL], qn[NPL];
    TokenIn nx{0.f, 0.f, 0.f};
    auto fetch = [&](int64_t t) {
        const int64_t kb = (t * Hk + hk) * Dk + col;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            kn[j] = load_any(k, kb + j, qk_dtype);
            qn[j] = load_any(q, kb + j, qk_dtype);
        }
        nx.g = load_any(g, t * Hv + h, g_dtype);
        nx.beta = load_any(beta, t * Hv + h, beta_dtype);
        nx.v = active ? load_any(v, (t * Hv + h) * Dv + row, v_dtype) : 0.f;
    };
    if (t0 < t1) fetch(t0);
    for (int64_t t = t0; t < t1; ++t) {
        float kk[NPL], qq[NPL];
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            kk[j] = kn[j];
            qq[j] = qn[j];
        }
        const TokenIn cur = nx;
        if (t + 1 < t1) fetch(t + 1);

        float sk = 0.f, sq = 0.f, kq = 0.f;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            sk += S[j] * kk[j];
            sq += S[j] * qq[j];
            kq += kk[j] * qq[j];
        }
        sk = group_sum<32>(sk);
        sq = group_sum<32>(sq);
        kq = group_sum<32>(kq);
        const float delta = (cur.v - cur.g * sk) * cur.beta;
        const float out = cur.g * sq + delta * kq;
#pragma unroll
        for (int j = 0; j < NPL; ++j) S[j] = cur.g * S[j] + delta * kk[j];
        if (active && l32 == 0) store_any(y, (t * Hv + h) * Dv + row, y_dtype, out);
    }
    if (active) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) store_any(state_out, sbase + j, state_dtype, S[j]);
    }
}

static int check_scan_args(const char* who, const void* q, const void* k, int qk_dtype,
                           const void* v, int v_dtype, const void* g, int g_dtype,
                           const void* beta, int beta_dtype, const void* state_in,
                           void* state_out, int state_dtype, void* y, int y_dtype,
                           const int32_t* cu, int N, int64_t T_total, int Hk, int Hv, int Dk,
                           int Dv) {
    GDN_REQUIRE(N > 0 && T_total >= 0 && Hk > 0 && Hv > 0 && Dk > 0 && Dv > 0,
                "%s: bad sizes", who);
    GDN_REQUIRE(Hv % Hk == 0, "%s: Hv=%d is not a multiple of Hk=%d", who, Hv, Hk);
    GDN_REQUIRE(valid_dtype(qk_dtype) && valid_dtype(v_dtype) && valid_dtype(g_dtype) &&
                    valid_dtype(beta_dtype) && valid_dtype(state_dtype) && valid_dtype(y_dtype),
                "%s: bad dtype", who);
    GDN_REQUIRE(cu || T_total % N == 0, "%s: T_total not divisible by N without cu_seqlens", who);
    GDN_REQUIRE(state_in && state_out, "%s: null state", who);
    GDN_REQUIRE(T_total == 0 || (q && k && v && g && beta && y), "%s: null pointer", who);
    return 0;
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_scan_reference(const void* q, const void* k, int qk_dtype, const void* v,
                                  int v_dtype, const void* g, int g_dtype, const void* beta,
                                  int beta_dtype, const void* state_in, void* state_out,
                                  int state_dtype, void* y, int y_dtype,
                                  const int32_t* cu_seqlens, int N, int64_t T_total, int Hk,
                                  int Hv, int Dk, int Dv, void* stream) {
    if (int rc = check_scan_args("gdn_scan_reference", q, k, qk_dtype, v, v_dtype, g, g_dtype,
                                 beta, beta_dtype, state_in, state_out, state_dtype, y, y_dtype,
                                 cu_seqlens, N, T_total, Hk, Hv, Dk, Dv))
        return rc;
    GDN_REQUIRE(Dk <= 256, "gdn_scan_reference: Dk=%d exceeds 256", Dk);
    const int64_t rows = int64_t(N) * Hv * Dv;
    const int threads = 64;
    const int64_t blocks = (rows + threads - 1) / threads;
    const int64_t L_uniform = cu_seqlens ? 0 : T_total / N;
    hipLaunchKernelGGL(scan_reference_kernel, dim3(unsigned(blocks)), dim3(threads), 0,
                       as_stream(stream), q, k, qk_dtype, v, v_dtype, g, g_dtype, beta,
                       beta_dtype, state_in, state_out, state_dtype, y, y_dtype, cu_seqlens, N,
                       L_uniform, Hk, Hv, Dk, Dv);
    return check_launch("gdn_scan_reference");
}

extern "C" int gdn_scan(const void* q, const void* k, int qk_dtype, const void* v, int v_dtype,
                        const void* g, int g_dtype, const void* beta, int beta_dtype,
                        const void* state_in, void* state_out, int state_dtype, void* y,
                        int y_dtype, const int32_t* cu_seqlens, int N, int64_t T_total, int Hk,
                        int Hv, int Dk, int Dv, void* stream) {
    if (int rc = check_scan_args("gdn_scan", q, k, qk_dtype, v, v_dtype, g, g_dtype, beta,
                                 beta_dtype, state_in, state_out, state_dtype, y, y_dtype,
                                 cu_seqlens, N, T_total, Hk, Hv, Dk, Dv))
        return rc;
    const int64_t tiles = (Dv + kScanRows - 1) / kScanRows;
    const int64_t blocks = int64_t(N) * Hv * tiles;
    const int64_t L_uniform = cu_seqlens ? 0 : T_total / N;
    hipStream_t s = as_stream(stream);
#define GDN_SCAN_LAUNCH(NPL)                                                                   \
    hipLaunchKernelGGL(scan_kernel<NPL>, dim3(unsigned(blocks)), dim3(kScanThreads), 0, s, q, k, \
                       qk_dtype, v, v_dtype, g, g_dtype, beta, beta_dtype, state_in, state_out, \
                       state_dtype, y, y_dtype, cu_seqlens, N, L_uniform, Hk, Hv, Dk, Dv)
    switch (Dk) {
        case 32: GDN_SCAN_LAUNCH(1); break;
        case 64: GDN_SCAN_LAUNCH(2); break;
        case 128: GDN_SCAN_LAUNCH(4); break;
        case 256: GDN_SCAN_LAUNCH(8); break;
        default:
            return fail(GDN_EUNSUPPORTED, "gdn_scan: Dk=%d not in {32, 64, 128, 256}", Dk);
    }
#undef GDN_SCAN_LAUNCH
    return check_launch("gdn_scan");
}
