// Prefill front-end: causal depthwise conv + SiLU + conv-state roll, then the
// q/k scaling, for N packed token runs (linear_attention.py:61-79,103-113).
//
// Blocks [0, T_total) each own one token: every channel's K-tap conv goes to
// LDS, then one wave per q/k head normalises. Blocks [T_total, T_total + N)
// each write one run's new conv state (the last K-1 rows of
// concat(state, tokens)), so conv_state_out must not overlap conv_state_in.
#include "gdn_common.h"
#include "gdn_host.h"

namespace gdn {

constexpr int kFrontThreads = 256;

template <class Act>
__global__ __launch_bounds__(kFrontThreads) void frontend_kernel(
    const typename Act::storage* __restrict__ qkv, const void* __restrict__ cs_in,
    int conv_dtype, typename Act::storage* __restrict__ cs_out, const float* __restrict__ w,
    const int32_t* __restrict__ cu, int N, int64_t T, int64_t L_uniform,
    typename Act::storage* __restrict__ qo, typename Act::storage* __restrict__ ko,
    typename Act::storage* __restrict__ vo, int Hk, int Hv, int Dk, int Dv, int K) {
    extern __shared__ float conv_out[];  // C floats
    const int C = 2 * Hk * Dk + Hv * Dv;
    const int64_t blk = blockIdx.x;
    const int tid = threadIdx.x;
    const int S = K - 1;  // conv state rows

    if (blk >= T) {
        // New conv state of one run: row j is concat index len + j.
        const int run = int(blk - T);
        if (run >= N) return;
        const int64_t start = cu ? cu[run] : run * L_uniform;
        const int64_t len = cu ? cu[run + 1] - cu[run] : L_uniform;
        for (int c = tid; c < C; c += kFrontThreads) {
            for (int j = 0; j < S; ++j) {
                const int64_t idx = len + j;
                const float x = idx < S
                    ? Act::round(load_any(cs_in, (int64_t(run) * S + idx) * C + c, conv_dtype))
                    : Act::load(qkv, (start + idx - S) * C + c);
                Act::store(cs_out, (int64_t(run) * S + j) * C + c, x);
            }
        }
        return;
    }

    const int64_t t = blk;
    const int run = cu ? find_run(cu, N, t) : int(t / L_uniform);
    const int64_t start = cu ? cu[run] : run * L_uniform;
    const int64_t pos = t - start;  // position inside the run
    for (int c = tid; c < C; c += kFrontThreads) {
        float acc = 0.f;
        for (int j = 0; j < K; ++j) {
            const int64_t idx = pos + j;  // index into concat(state, run tokens)
            const float x = idx < S
                ? Act::round(load_any(cs_in, (int64_t(run) * S + idx) * C + c, conv_dtype))
                : Act::load(qkv, (start + idx - S) * C + c);
            acc += Act::round(w[int64_t(c) * K + j]) * x;
        }
        acc = Act::round(acc);
        conv_out[c] = Act::round(silu(acc));
    }
    __syncthreads();

    const int wave = tid / kWave, lane = tid % kWave;
    const float inv = 1.f / sqrtf(float(Dk));
    const float scale_q = Act::round(inv * inv), scale_k = Act::round(inv);
    for (int head = wave; head < 2 * Hk; head += kFrontThreads / kWave) {
        const float* src = conv_out + head * Dk;
        float ss = 0.f;
        for (int e = lane; e < Dk; e += kWave) ss += src[e] * src[e];
        ss = group_sum<kWave>(ss);
        const float r = 1.f / sqrtf(ss / float(Dk) + 1e-6f);
        const bool is_q = head < Hk;
        const float sc = is_q ? scale_q : scale_k;
        typename Act::storage* dst = is_q ? qo + (t * Hk + head) * Dk : ko + (t * Hk + head - Hk) * Dk;
        for (int e = lane; e < Dk; e += kWave) Act::store(dst, e, sc * Act::round(src[e] * r));
    }
    const float* vsrc = conv_out + 2 * Hk * Dk;
    for (int e = tid; e < Hv * Dv; e += kFrontThreads) Act::store(vo, t * Hv * Dv + e, vsrc[e]);
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_frontend(const void* qkv, const void* conv_state_in, void* conv_state_out,
                            int conv_dtype, const float* conv_weight, const int32_t* cu_seqlens,
                            int N, int64_t T_total, void* q_out, void* k_out, void* v_out, int Hk,
                            int Hv, int Dk, int Dv, int K, int act_dtype, void* stream) {
    GDN_REQUIRE(N > 0 && T_total >= 0 && Hk > 0 && Hv > 0 && Dk > 0 && Dv > 0 && K >= 1,
                "gdn_frontend: bad sizes");
    GDN_REQUIRE(Hv % Hk == 0, "gdn_frontend: Hv=%d is not a multiple of Hk=%d", Hv, Hk);
    GDN_REQUIRE(valid_dtype(conv_dtype), "gdn_frontend: bad conv dtype");
    GDN_REQUIRE(act_dtype == GDN_F32 || act_dtype == GDN_BF16,
                "gdn_frontend: activations must be float32 or bfloat16");
    GDN_REQUIRE(cu_seqlens || T_total % N == 0,
                "gdn_frontend: T_total=%lld not divisible by N=%d without cu_seqlens",
                (long long)T_total, N);
    const int64_t C = 2LL * Hk * Dk + int64_t(Hv) * Dv;
    GDN_REQUIRE(C * 4 <= 64 * 1024, "gdn_frontend: conv_dim %lld exceeds the LDS tile", (long long)C);
    const int64_t S = K - 1;
    if (S > 0) {
        GDN_REQUIRE(conv_state_in && conv_state_out, "gdn_frontend: null conv state");
        GDN_REQUIRE(!overlaps(conv_state_in, N * S * C * dtype_size(conv_dtype), conv_state_out,
                              N * S * C * dtype_size(act_dtype)),
                    "gdn_frontend: conv_state_out overlaps conv_state_in");
    }
    if (T_total == 0 && S == 0) return 0;
    GDN_REQUIRE(conv_weight && (T_total == 0 || (qkv && q_out && k_out && v_out)),
                "gdn_frontend: null pointer");
    const int64_t L_uniform = cu_seqlens ? 0 : T_total / N;
    const int64_t blocks = T_total + (S > 0 ? N : 0);
    if (blocks == 0) return 0;
    const size_t lds = size_t(C) * sizeof(float);
    if (act_dtype == GDN_F32) {
        hipLaunchKernelGGL(frontend_kernel<ActF32>, dim3(unsigned(blocks)), dim3(kFrontThreads),
                           lds, as_stream(stream), static_cast<const float*>(qkv), conv_state_in,
                           conv_dtype, static_cast<float*>(conv_state_out), conv_weight,
                           cu_seqlens, N, T_total, L_uniform, static_cast<float*>(q_out),
                           static_cast<float*>(k_out), static_cast<float*>(v_out), Hk, Hv, Dk,
                           Dv, K);
    } else {
        hipLaunchKernelGGL(frontend_kernel<ActBF16>, dim3(unsigned(blocks)), dim3(kFrontThreads),
                           lds, as_stream(stream), static_cast<const uint16_t*>(qkv),
                           conv_state_in, conv_dtype, static_cast<uint16_t*>(conv_state_out),
                           conv_weight, cu_seqlens, N, T_total, L_uniform,
                           static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out),
                           static_cast<uint16_t*>(v_out), Hk, Hv, Dk, Dv, K);
    }
    return check_launch("gdn_frontend");
}
