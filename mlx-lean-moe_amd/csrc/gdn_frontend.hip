// Prefill front-end: causal depthwise conv + SiLU + conv-state roll, then the
// q/k scaling, for N packed token runs (linear_attention.py:61-79,103-113).
//
// Two kernels. The tiled one covers the production shape (Dk = Dv = 128,
// K = 4, bf16 activations, 16-byte aligned operands): a wave holds four
// 128-channel groups (q, k or v heads) of one token, 8 channels a lane, and
// walks a tile of 4-16 tokens with the previous three input rows in registers, so
// each qkv row is read once per tile plus a three-row halo, with 16-byte
// loads and stores; the q/k RMS norm is a 16-lane DPP sum. The general
// one (any head size and K) gives each token a block: every channel's K-tap
// conv goes to LDS, then one wave per q/k head normalises. In both, extra
// blocks each write one run's new conv state (the last K-1 rows of
// concat(state, tokens)), so conv_state_out must not overlap conv_state_in.
#include <type_traits>

#include "gdn_common.h"
#include "gdn_conv.h"
#include "gdn_host.h"

namespace gdn {

constexpr int kFrontThreads = 256;

// Row j of a run's new conv state is row len + j of concat(state, tokens).
template <class Act>
GDN_DEV void write_conv_state(const typename Act::storage* __restrict__ qkv, int64_t qs,
                              const void* __restrict__ cs_in, int conv_dtype,
                              typename Act::storage* __restrict__ cs_out,
                              const int32_t* __restrict__ cu, int run, int64_t L_uniform, int C,
                              int S) {
    const int64_t start = cu ? cu[run] : run * L_uniform;
    const int64_t len = cu ? cu[run + 1] - cu[run] : L_uniform;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        for (int j = 0; j < S; ++j) {
            const int64_t idx = len + j;
            const float x = idx < S
                ? Act::round(load_any(cs_in, (int64_t(run) * S + idx) * C + c, conv_dtype))
                : Act::load(qkv, (start + idx - S) * qs + c);
            Act::store(cs_out, (int64_t(run) * S + j) * C + c, x);
        }
    }
}

template <class Act>
__global__ __launch_bounds__(kFrontThreads) void frontend_kernel(
    const typename Act::storage* __restrict__ qkv, int64_t qs, const void* __restrict__ cs_in,
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
        const int run = int(blk - T);
        if (run < N) write_conv_state<Act>(qkv, qs, cs_in, conv_dtype, cs_out, cu, run, L_uniform, C, S);
        return;
    }

    const int64_t t = blk;
    const int run = cu ? find_run(cu, N, t) : int(t / L_uniform);
    const int64_t start = cu ? cu[run] : run * L_uniform;
    const int64_t pos = t - start;  // position inside the run
    // the conv and SiLU of each channel, with the tiled kernel's instruction
    // sequence (conv_chain, silu_act; for float32 that is the decode step's)
    for (int c = tid; c < C; c += kFrontThreads) {
        float acc[1] = {Act::round(conv_chain(K, [&](int j) {
            const int64_t idx = pos + j;  // index into concat(state, run tokens)
            const float x = idx < S
                ? Act::round(load_any(cs_in, (int64_t(run) * S + idx) * C + c, conv_dtype))
                : Act::load(qkv, (start + idx - S) * qs + c);
            return float2{Act::round(w[int64_t(c) * K + j]), x};
        }))};
        silu_act<Act::code>(acc);
        conv_out[c] = Act::round(acc[0]);
    }
    __syncthreads();

    // the q/k scaling: 128-wide bf16 heads with the tiled kernels' rms_norm8
    // (lane l takes channels 8 (l % 16) .. + 7, the wave's four DPP rows the
    // same head, the first storing it); others in double, each value rounded
    // once (rms_rr), as the decode step scales them
    const int wave = tid / kWave, lane = tid % kWave;
    const float inv = 1.f / sqrtf(float(Dk));
    const float scale_q = Act::round(inv * inv), scale_k = Act::round(inv);
    for (int head = wave; head < 2 * Hk; head += kFrontThreads / kWave) {
        const float* src = conv_out + head * Dk;
        const bool is_q = head < Hk;
        const float sc = is_q ? scale_q : scale_k;
        typename Act::storage* dst = is_q ? qo + (t * Hk + head) * Dk : ko + (t * Hk + head - Hk) * Dk;
        if (Act::code == GDN_BF16 && Dk == 128) {
            const int c8 = 8 * (lane & 15);
            float o[8], n[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = src[c8 + e];
            rms_norm8(o, n);
            if (lane < 16) {
#pragma unroll
                for (int e = 0; e < 8; ++e) Act::store(dst, c8 + e, sc * n[e]);
            }
        } else {
            double ss = 0.0;
            for (int e = lane; e < Dk; e += kWave) ss = fma(double(src[e]), double(src[e]), ss);
            const double rr = rms_rr(group_sum<kWave>(ss), Dk);
            for (int e = lane; e < Dk; e += kWave)
                Act::store(dst, e, sc * round_once(double(src[e]) * rr, Act::code));
        }
    }
    const float* vsrc = conv_out + 2 * Hk * Dk;
    for (int e = tid; e < Hv * Dv; e += kFrontThreads) Act::store(vo, t * Hv * Dv + e, vsrc[e]);
}


constexpr int kMaxTileTokens = 16;  // tokens a wave walks, at most
constexpr int kTileWaves = 4;    // waves a block, four channel groups each

constexpr int kStateChunk = kTileWaves * kWave * 8;  // conv-state elements a block writes

// Tiles of kTileTokens = TT tokens (16, or 8 or 4 for short inputs).
// grid (n_state + n_tiles, ceil(G / 16)) for G = 2 Hk + Hv channel groups of
// 128. The first n_state columns write the runs' new conv states, flattened
// to N (K-1) C elements, kStateChunk a block (8 independent elements a
// thread; dispatched first, they overlap the tiles); block (n_state + x, y)
// covers tokens [TT x, TT x + TT) of groups [16 y, 16 y + 16).
//
// The three-row window holds rows t-3 .. t-1 of concat(run's conv state,
// run's tokens) for the token t in hand: it is loaded so at the tile's first
// token and reloaded from the conv state where a run starts inside the tile,
// and each token shifts itself in.
template <int kConvDt, int kTileTokens>
__global__ __launch_bounds__(kTileWaves * kWave) void frontend_tiled_kernel(
    const uint16_t* __restrict__ qkv, int64_t qs, const void* __restrict__ cs_in,
    uint16_t* __restrict__ cs_out, const float* __restrict__ w, const int32_t* __restrict__ cu,
    int N, int64_t T, int64_t L_uniform, int n_state, uint16_t* __restrict__ qo,
    uint16_t* __restrict__ ko, uint16_t* __restrict__ vo, int Hk, int Hv) {
    constexpr int D = 128, K = 4, S = K - 1;
    const int G = 2 * Hk + Hv;
    const int C = G * D;
    if (int(blockIdx.x) < n_state) {
        const int64_t total = int64_t(N) * S * C;
        const int64_t first = (int64_t(blockIdx.x) * gridDim.y + blockIdx.y) * kStateChunk + threadIdx.x;
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // all loads first: they do not wait on each other
            const int64_t e = first + int64_t(i) * kTileWaves * kWave;
            if (e < total) {
                const int run = int(e / (int64_t(S) * C));
                const int j = int(e / C % S), c = int(e % C);
                const int64_t start = cu ? cu[run] : run * L_uniform;
                const int64_t idx = (cu ? cu[run + 1] - cu[run] : L_uniform) + j;  // in concat(state, run)
                x[i] = idx < S ? round_bf16(load_any(cs_in, (int64_t(run) * S + idx) * C + c, kConvDt))
                               : ActBF16::load(qkv, (start + idx - S) * qs + c);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t e = first + int64_t(i) * kTileWaves * kWave;
            if (e < total) ActBF16::store(cs_out, e, x[i]);
        }
        return;
    }
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int g0 = (int(blockIdx.y) * kTileWaves + wave) * 4;  // the wave's first group
    if (g0 >= G) return;  // the whole wave idles; the kernel has no barrier
    const int g = g0 + lane / 16;
    const bool live = g < G;
    const int c0 = (live ? g : G - 1) * D + (lane % 16) * 8;  // this lane's 8 channels
    const int64_t t0 = (int64_t(blockIdx.x) - n_state) * kTileTokens;

    // the tile's rows, kAhead in flight (the last tile's missing ones repeat
    // row T-1, unused)
    constexpr int kAhead = kTileTokens < 8 ? kTileTokens : 8;
    const auto row_at = [&](int i) {
        const int64_t t = t0 + i < T ? t0 + i : T - 1;
        return *reinterpret_cast<const uint4*>(qkv + t * qs + c0);
    };
    uint4 raw[kAhead];
#pragma unroll
    for (int i = 0; i < kAhead; ++i) raw[i] = row_at(i);
    int run = cu ? find_run(cu, N, t0) : int(t0 / L_uniform);
    int64_t start = cu ? cu[run] : run * L_uniform;
    int64_t next = cu ? cu[run + 1] : start + L_uniform;
    float win[S][8];
#pragma unroll
    for (int j = 0; j < S; ++j) {
        const int64_t row = t0 - S + j;
        if (row >= start) {
            unpack8(*reinterpret_cast<const uint4*>(qkv + row * qs + c0), win[j]);
        } else {  // concat index row - start + S of the run's conv state
            load_state8<kConvDt>(cs_in, (int64_t(run) * S + (row - start + S)) * C + c0, win[j]);
        }
    }
    float wr[8][K];
    load_conv_w8(w, c0, wr);

    const float inv = 1.f / sqrtf(float(D));
    const float sc = g < Hk ? round_bf16(inv * inv) : round_bf16(inv);
    const bool is_v = g >= 2 * Hk;
    // whether the wave holds a q or k head (uniform: a wave may also hold v
    // heads when Hk is not a multiple of 4; their lanes keep o)
    const bool qk_wave = __builtin_amdgcn_readfirstlane(int(g0 < 2 * Hk)) != 0;
    uint16_t* dst = g < Hk ? qo + int64_t(g) * D
                  : !is_v ? ko + int64_t(g - Hk) * D
                          : vo + int64_t(g - 2 * Hk) * D;
    const int64_t dst_row = is_v ? int64_t(Hv) * D : int64_t(Hk) * D;
    dst += (lane % 16) * 8;

#pragma unroll
    for (int i = 0; i < kTileTokens; ++i) {
        const int64_t t = t0 + i;
        if (t < T && t >= next) {  // a run starts at t (uniform): its conv state is the window
            run = cu ? find_run(cu, N, t) : int(t / L_uniform);
            start = t;
            next = cu ? cu[run + 1] : t + L_uniform;
#pragma unroll
            for (int j = 0; j < S; ++j)
                load_state8<kConvDt>(cs_in, (int64_t(run) * S + j) * C + c0, win[j]);
        }
        float x[8];
        unpack8(raw[i % kAhead], x);
        if (i + kAhead < kTileTokens) raw[i % kAhead] = row_at(i + kAhead);
        float o[8];
        conv_silu8(wr, win, x, o);
        if (qk_wave) {  // q and k heads: scaled RMS norm (v lanes keep o)
            float n[8];
            rms_norm8(o, n);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = is_v ? o[e] : sc * n[e];
        }
        if (live && t < T) *reinterpret_cast<uint4*>(dst + t * dst_row) = pack8(o);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            win[0][e] = win[1][e];
            win[1][e] = win[2][e];
            win[2][e] = x[e];
        }
    }
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_frontend(const void* qkv, int64_t qkv_stride, const void* conv_state_in, void* conv_state_out,
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
    GDN_REQUIRE(qkv_stride >= C, "gdn_frontend: qkv_stride %lld below conv_dim %lld",
                (long long)qkv_stride, (long long)C);
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
    const auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (act_dtype == GDN_BF16 && Dk == 128 && Dv == 128 && K == 4 && T_total > 0 && aligned(qkv) &&
        qkv_stride % 8 == 0 &&
        aligned(conv_state_in) && aligned(conv_weight) && aligned(q_out) && aligned(k_out) &&
        aligned(v_out)) {
        const int G = 2 * Hk + Hv;
        const int gy = (G + 4 * kTileWaves - 1) / (4 * kTileWaves);
        // tiles of 16 tokens, or of 8 or 4 where that leaves under 1024
        // workgroups (a wave walks its tile's tokens one after another)
        int tile = kMaxTileTokens;
        while (tile > 4 && (T_total + tile - 1) / tile * gy < 1024) tile /= 2;
        const int64_t n_tiles = (T_total + tile - 1) / tile;
        const int64_t chunks = (int64_t(N) * S * C + kStateChunk - 1) / kStateChunk;
        const int64_t n_state = (chunks + gy - 1) / gy;
        const int64_t gx = n_state + n_tiles;
        GDN_REQUIRE(gx < (1LL << 31) / (kTileWaves * kWave) && gy < 65536,
                    "gdn_frontend: %lld tokens exceed the grid", (long long)T_total);
        using Kernel = void (*)(const uint16_t*, int64_t, const void*, uint16_t*, const float*, const int32_t*,
                                int, int64_t, int64_t, int, uint16_t*, uint16_t*, uint16_t*, int, int);
        const auto pick = [&](auto tt) -> Kernel {
            constexpr int TT = decltype(tt)::value;
            return conv_dtype == GDN_F32    ? frontend_tiled_kernel<GDN_F32, TT>
                   : conv_dtype == GDN_BF16 ? frontend_tiled_kernel<GDN_BF16, TT>
                                            : frontend_tiled_kernel<GDN_F16, TT>;
        };
        const Kernel kern = tile == 16 ? pick(std::integral_constant<int, 16>{})
                            : tile == 8 ? pick(std::integral_constant<int, 8>{})
                                        : pick(std::integral_constant<int, 4>{});
        hipLaunchKernelGGL(kern, dim3(unsigned(gx), unsigned(gy)), dim3(kTileWaves * kWave), 0,
                           as_stream(stream), static_cast<const uint16_t*>(qkv), qkv_stride, conv_state_in,
                           static_cast<uint16_t*>(conv_state_out), conv_weight, cu_seqlens, N,
                           T_total, L_uniform, int(n_state), static_cast<uint16_t*>(q_out),
                           static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out), Hk, Hv);
        return check_launch("gdn_frontend");
    }
    const int64_t blocks = T_total + (S > 0 ? N : 0);
    if (blocks == 0) return 0;
    const size_t lds = size_t(C) * sizeof(float);
    if (act_dtype == GDN_F32) {
        hipLaunchKernelGGL(frontend_kernel<ActF32>, dim3(unsigned(blocks)), dim3(kFrontThreads),
                           lds, as_stream(stream), static_cast<const float*>(qkv), qkv_stride, conv_state_in,
                           conv_dtype, static_cast<float*>(conv_state_out), conv_weight,
                           cu_seqlens, N, T_total, L_uniform, static_cast<float*>(q_out),
                           static_cast<float*>(k_out), static_cast<float*>(v_out), Hk, Hv, Dk,
                           Dv, K);
    } else {
        hipLaunchKernelGGL(frontend_kernel<ActBF16>, dim3(unsigned(blocks)), dim3(kFrontThreads),
                           lds, as_stream(stream), static_cast<const uint16_t*>(qkv), qkv_stride,
                           conv_state_in, conv_dtype, static_cast<uint16_t*>(conv_state_out),
                           conv_weight, cu_seqlens, N, T_total, L_uniform,
                           static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out),
                           static_cast<uint16_t*>(v_out), Hk, Hv, Dk, Dv, K);
    }
    return check_launch("gdn_frontend");
}
