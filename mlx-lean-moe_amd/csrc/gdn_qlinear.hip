// Affine-quantized linear layers (MLX's packing) for the layer's input and
// output projections.
//
// The reference runs them as mx.quantized_matmul(x, weight, scales, biases,
// group_size, bits, mode="affine") (model/moe_block.py:44-55, called from
// model/qwen3_5/linear_attention.py:96-101,125). Weight layout (N, K):
// `weight` is uint32 (N, K * bits / 32) with element k of a row at bits
// [bits * (k % per_word), +bits) of word k / per_word (least significant
// first); `scales` and `biases` are (N, K / group_size) in the model dtype;
// w[n][k] = scales[n][g] * q + biases[n][g], g = k / group_size.
//
// gdn_quantized_matmul: y = x W^T for bf16 x on v_mfma_f32_16x16x32_bf16.
// Each K step of 64 dequantizes a BN x 64 tile of W to bf16 in LDS (the
// scale * q + bias product is exact in float32, rounded once to bf16: the
// weights mx.dequantize yields) next to a BM x 64 tile of x; fp32
// accumulation. Loads of step s + 1 are issued before step s's MFMAs.
// gdn_dequantize: the dense weights, for dtypes the MFMA kernel does not take.
#include "gdn_common.h"
#include "gdn_host.h"

namespace gdn {
namespace {

constexpr int kBK = 64;          // K per pipeline step
constexpr int kTS = kBK + 8;     // bf16 row stride of the LDS tiles

GDN_DEV f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int kBits>
struct Packing {
    static constexpr int per_word = 32 / kBits;
    static constexpr uint32_t mask = (1u << kBits) - 1u;
};

// One thread's share of a K step of W: 32 consecutive k of one row n
// (16 bytes of 4-bit codes, 32 of 8-bit), dequantized to bf16.
template <int kBits, class SB>
struct WSlice {
    uint4 words[kBits / 4];
    typename SB::storage scale, bias;  // raw: converted only when dequantizing, so that
                                       // the loads are not waited for at issue

    GDN_DEV void load(const uint32_t* w, const typename SB::storage* scales,
                      const typename SB::storage* biases, int64_t row, int64_t k0, int K,
                      int group_size) {
        const int64_t wpr = int64_t(K) / Packing<kBits>::per_word;  // words per row
        const uint4* src = reinterpret_cast<const uint4*>(w + row * wpr + k0 / Packing<kBits>::per_word);
#pragma unroll
        for (int i = 0; i < kBits / 4; ++i) words[i] = src[i];
        const int64_t gi = row * (K / group_size) + k0 / group_size;
        scale = scales[gi];
        bias = biases[gi];
    }

    // bf16 weights of the 32 k, as four 8-element vectors.
    GDN_DEV void dequant(u16x8 (&out)[4]) const {
        const uint32_t* wd = reinterpret_cast<const uint32_t*>(words);
        const float s = SB::load(&scale, 0), b = SB::load(&bias, 0);
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const uint32_t word = wd[j / Packing<kBits>::per_word];
            const uint32_t q = (word >> (kBits * (j % Packing<kBits>::per_word))) & Packing<kBits>::mask;
            out[j / 8][j % 8] = f32_to_bf16_bits(__builtin_fmaf(s, float(q), b));
        }
    }
};

// y[m][n] = sum_k x[m][k] w[n][k]. 256 threads, waves 2 x 2 over the
// BM x BN tile. Rows m >= M and n >= N are read clamped and never stored.
template <int BM, int BN, int kBits, class SB, class Y>
__global__ __launch_bounds__(256) void qlinear_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const typename SB::storage* __restrict__ scales, const typename SB::storage* __restrict__ biases,
    typename Y::storage* __restrict__ y, int M, int N, int K, int group_size) {
    static_assert(BN <= 128 && BM * 8 % 256 == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][BM * kTS];
    __shared__ __attribute__((aligned(16))) uint16_t ws[2][BN * kTS];

    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 16, TN = WN / 16;
    constexpr int XLOADS = BM * 8 / 256;  // 16-byte pieces of the x tile per thread
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, lr = l & 15, lq = l >> 4;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int wm = (wv >> 1) * WM, wn = (wv & 1) * WN;

    // the thread's W slice: row n0 + tid / 2, k half tid % 2; with BN < 128
    // the threads past the tile repeat a slice of the tile (same loads, same
    // values, same LDS words), so that loads and stores stay unconditional: a
    // conditional consumer lets the compiler sink the prefetch into it
    const int wrow = (tid >> 1) % BN, whalf = tid & 1;
    const int64_t wn_row = n0 + wrow < N ? n0 + wrow : N - 1;

    u16x8 xr[XLOADS];
    WSlice<kBits, SB> wsl;
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < XLOADS; ++i) {
            const int idx = tid + 256 * i, row = idx >> 3, seg = idx & 7;
            const int64_t m = m0 + row < M ? m0 + row : M - 1;
            xr[i] = *reinterpret_cast<const u16x8*>(x + m * K + k0 + 8 * seg);
        }
        wsl.load(w, scales, biases, wn_row, k0 + 32 * whalf, K, group_size);
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XLOADS; ++i) {
            const int idx = tid + 256 * i, row = idx >> 3, seg = idx & 7;
            *reinterpret_cast<u16x8*>(&xs[buf][row * kTS + 8 * seg]) = xr[i];
        }
        u16x8 dq[4];
        wsl.dequant(dq);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<u16x8*>(&ws[buf][wrow * kTS + 32 * whalf + 8 * j]) = dq[j];
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int steps = K / kBK;
    fetch(0);
    stage(0);
    __syncthreads();
    for (int s = 0; s < steps; ++s) {
        const int buf = s & 1;
        fetch(s + 1 < steps ? (s + 1) * kBK : s * kBK);  // the last step re-reads itself
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the MFMAs
#pragma unroll
        for (int kb = 0; kb < kBK / 32; ++kb) {
            bf16x8 af[TM], bfr[TN];
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[a] = *reinterpret_cast<const bf16x8*>(&xs[buf][(wm + 16 * a + lr) * kTS + 32 * kb + 8 * lq]);
#pragma unroll
            for (int b = 0; b < TN; ++b)
                bfr[b] = *reinterpret_cast<const bf16x8*>(&ws[buf][(wn + 16 * b + lr) * kTS + 32 * kb + 8 * lq]);
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) acc[a][b] = mfma_bf16(af[a], bfr[b], acc[a][b]);
        }
        __builtin_amdgcn_sched_barrier(0);  // and the loaded values' first use after them
        stage(buf ^ 1);  // unconditional: the last step stages into the idle buffer
        __syncthreads();
    }

    // acc[a][b][i] = y[m0 + wm + 16a + 4(l/16) + i][n0 + wn + 16b + l%16]
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int n = n0 + wn + 16 * b + lr;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + wm + 16 * a + 4 * lq + i;
                if (m < M && n < N) Y::store(y, int64_t(m) * N + n, acc[a][b][i]);
            }
        }
}

// Small M (decode, M <= 64): weight-stationary. One 1024-thread workgroup
// per 64 output columns over the whole K: each thread requests its share of
// the packed weights for every K step (16 consecutive k of one column per
// step) at the start, and the workgroup's scales and biases go to LDS with
// 16-byte loads, so the HBM stream is issued at once; x then streams from L2
// in steps of 256 k through double-buffered LDS, where each step's weights
// are also dequantized. Wave w computes the 16 x 16 output tile (w / 4,
// w % 4) of the 64 x 64 block. kSteps = K / 256; the 64 columns' K /
// group_size scales (and as many biases) must fit kSmallSBBytes each.
constexpr int kSmallBK = 256;
constexpr int kSmallTS = kSmallBK + 8;
constexpr int kSmallSBBytes = 14336;  // LDS bytes for scales (and again for biases)

template <int kBits, int kSteps, class SB, class Y>
__global__ __launch_bounds__(1024) void qlinear_small_m_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const typename SB::storage* __restrict__ scales, const typename SB::storage* __restrict__ biases,
    typename Y::storage* __restrict__ y, int M, int N, int K, int group_size) {
    typedef uint32_t wword_t __attribute__((ext_vector_type(kBits / 2)));  // 16 codes
    using sb_t = typename SB::storage;
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][64 * kSmallTS];
    __shared__ __attribute__((aligned(16))) uint16_t ws[2][64 * kSmallTS];
    __shared__ __attribute__((aligned(16))) sb_t sbs[2][kSmallSBBytes / sizeof(sb_t)];  // [column][group]

    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, lr = l & 15, lq = l >> 4;
    const int n0 = blockIdx.x * 64;
    // weight share: column n0 + tid / 16, k = 256 s + 16 (tid % 16) .. +15
    const int wc = tid >> 4, wk = 16 * (tid & 15);
    const int64_t wrow = n0 + wc < N ? n0 + wc : N - 1;
    const int64_t wpr = int64_t(K) / Packing<kBits>::per_word;
    const int gpr = K / group_size;

    // x share per step: row tid / 16 (clamped to M - 1), k 8 (tid % 16) + {0, 128} .. +7
    const int xr = tid >> 4, xk = 8 * (tid & 15);
    const int64_t xrow = xr < M ? xr : M - 1;
    u16x8 xv[2][2];
    auto fetch_x = [&](int s, u16x8 (&v)[2]) {
        const uint16_t* src = x + xrow * K + kSmallBK * s + xk;
        v[0] = *reinterpret_cast<const u16x8*>(src);
        v[1] = *reinterpret_cast<const u16x8*>(src + 128);
    };
    auto stage_x = [&](int buf, const u16x8 (&v)[2]) {
        *reinterpret_cast<u16x8*>(&xs[buf][xr * kSmallTS + xk]) = v[0];
        *reinterpret_cast<u16x8*>(&xs[buf][xr * kSmallTS + xk + 128]) = v[1];
    };

    // Scales and biases of the 64 columns are one contiguous span of 64
    // gpr entries each, loaded in 16-byte pieces, at most two per thread
    // (2 kSmallSBBytes / 16 <= 2048). They are requested first so that
    // waiting for them does not wait for the weight stream. Pieces past the
    // end of the arrays (columns >= N, whose outputs are not stored) read
    // the last piece instead; threads past the last piece repeat it.
    constexpr int per_piece = 16 / int(sizeof(sb_t));
    const int span_pieces = 64 * gpr / per_piece;
    const int64_t base_piece = int64_t(n0) * gpr / per_piece, last_piece = int64_t(N) * gpr / per_piece - 1;
    int pdst[2];
    uint4 pv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int p = tid + 1024 * i;
        p = p < 2 * span_pieces ? p : 2 * span_pieces - 1;
        const int which = p >= span_pieces, o = p - which * span_pieces;
        const int64_t gp = base_piece + o < last_piece ? base_piece + o : last_piece;
        pv[i] = *reinterpret_cast<const uint4*>((which ? biases : scales) + gp * per_piece);
        pdst[i] = which * (kSmallSBBytes / 16) + o;
    }
    fetch_x(0, xv[0]);
    if (kSteps > 1) fetch_x(1, xv[1]);
    wword_t wq[kSteps];
#pragma unroll
    for (int s = 0; s < kSteps; ++s)
        wq[s] = *reinterpret_cast<const wword_t*>(w + wrow * wpr + (kSmallBK * s + wk) / Packing<kBits>::per_word);
#pragma unroll
    for (int i = 0; i < 2; ++i) reinterpret_cast<uint4*>(&sbs[0][0])[pdst[i]] = pv[i];
    __syncthreads();
    auto stage_w = [&](int buf, int s) {
        const int g = (kSmallBK * s + wk) / group_size;
        const float sf = SB::load(&sbs[0][wc * gpr + g], 0), bf = SB::load(&sbs[1][wc * gpr + g], 0);
        const uint32_t* words = reinterpret_cast<const uint32_t*>(&wq[s]);
        u16x8 dq[2];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t q = (words[j / Packing<kBits>::per_word] >> (kBits * (j % Packing<kBits>::per_word))) &
                               Packing<kBits>::mask;
            dq[j / 8][j % 8] = f32_to_bf16_bits(__builtin_fmaf(sf, float(q), bf));
        }
        *reinterpret_cast<u16x8*>(&ws[buf][wc * kSmallTS + wk]) = dq[0];
        *reinterpret_cast<u16x8*>(&ws[buf][wc * kSmallTS + wk + 8]) = dq[1];
    };

    const int tm = wv >> 2, tn = wv & 3;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    stage_x(0, xv[0]);
    stage_w(0, 0);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        const int buf = s & 1;
        if (s + 2 < kSteps) fetch_x(s + 2, xv[s & 1]);
#pragma unroll
        for (int kb = 0; kb < kSmallBK / 32; ++kb) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(&xs[buf][(16 * tm + lr) * kSmallTS + 32 * kb + 8 * lq]);
            const bf16x8 b = *reinterpret_cast<const bf16x8*>(&ws[buf][(16 * tn + lr) * kSmallTS + 32 * kb + 8 * lq]);
            acc = mfma_bf16(a, b, acc);
        }
        if (s + 1 < kSteps) {
            stage_x(buf ^ 1, xv[(s + 1) & 1]);
            stage_w(buf ^ 1, s + 1);
        }
        __syncthreads();
    }
    const int n = n0 + 16 * tn + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 16 * tm + 4 * lq + i;
        if (m < M && n < N) Y::store(y, int64_t(m) * N + n, acc[i]);
    }
}

template <int kBits, class SB, class Y>
int launch_small_m(const void* x, const uint32_t* w, const void* scales, const void* biases, void* y,
                   int M, int N, int K, int group_size, hipStream_t s) {
    const dim3 grid(unsigned((N + 63) / 64));
#define GDN_SMALL(STEPS)                                                                            \
    hipLaunchKernelGGL((qlinear_small_m_kernel<kBits, STEPS, SB, Y>), grid, dim3(1024), 0, s,          \
                       static_cast<const uint16_t*>(x), w,                                          \
                       static_cast<const typename SB::storage*>(scales),                            \
                       static_cast<const typename SB::storage*>(biases),                            \
                       static_cast<typename Y::storage*>(y), M, N, K, group_size)
    switch (K / kSmallBK) {
        case 1: GDN_SMALL(1); break;
        case 2: GDN_SMALL(2); break;
        case 4: GDN_SMALL(4); break;
        case 8: GDN_SMALL(8); break;
        case 16: GDN_SMALL(16); break;
        default: return -1;
    }
#undef GDN_SMALL
    return check_launch("gdn_quantized_matmul");
}

template <int kBits, class SB, class O>
__global__ void dequantize_kernel(const uint32_t* __restrict__ w, const typename SB::storage* __restrict__ scales,
                                  const typename SB::storage* __restrict__ biases,
                                  typename O::storage* __restrict__ out, int N, int K, int group_size) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;  // one word
    const int64_t wpr = K / Packing<kBits>::per_word;
    if (i >= int64_t(N) * wpr) return;
    const int64_t n = i / wpr, k0 = (i % wpr) * Packing<kBits>::per_word;
    const int64_t gi = n * (K / group_size) + k0 / group_size;
    const float s = SB::load(scales, gi), b = SB::load(biases, gi);
    const uint32_t word = w[i];
#pragma unroll
    for (int j = 0; j < Packing<kBits>::per_word; ++j) {
        const uint32_t q = (word >> (kBits * j)) & Packing<kBits>::mask;
        O::store(out, n * K + k0 + j, __builtin_fmaf(s, float(q), b));
    }
}

template <int BM, int BN, int kBits, class SB, class Y>
int launch_qlinear(const void* x, const uint32_t* w, const void* scales, const void* biases, void* y,
                   int M, int N, int K, int group_size, hipStream_t s) {
    const dim3 grid(unsigned((N + BN - 1) / BN), unsigned((M + BM - 1) / BM));
    hipLaunchKernelGGL((qlinear_kernel<BM, BN, kBits, SB, Y>), grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), w,
                       static_cast<const typename SB::storage*>(scales),
                       static_cast<const typename SB::storage*>(biases),
                       static_cast<typename Y::storage*>(y), M, N, K, group_size);
    return check_launch("gdn_quantized_matmul");
}

// Kernel choice: M <= 64 (decode) takes the weight-stationary kernel when
// K / 256 is 1, 2, 4, 8 or 16 (hidden sizes up to 4096), else 64 x 32 tiles;
// larger M takes 128 x 128 tiles.
template <int kBits, class SB, class Y>
int dispatch_qlinear(const void* x, const uint32_t* w, const void* scales, const void* biases,
                     void* y, int M, int N, int K, int group_size, hipStream_t s) {
    if (M <= 64) {
        const int ks = K / kSmallBK;
        if (K % kSmallBK == 0 && (ks == 1 || ks == 2 || ks == 4 || ks == 8 || ks == 16) &&
            64 * (K / group_size) * int(sizeof(typename SB::storage)) <= kSmallSBBytes &&
            int64_t(N) * (K / group_size) * int(sizeof(typename SB::storage)) % 16 == 0 &&
            reinterpret_cast<uintptr_t>(scales) % 16 == 0 && reinterpret_cast<uintptr_t>(biases) % 16 == 0)
            return launch_small_m<kBits, SB, Y>(x, w, scales, biases, y, M, N, K, group_size, s);
        return launch_qlinear<64, 32, kBits, SB, Y>(x, w, scales, biases, y, M, N, K, group_size, s);
    }
    return launch_qlinear<128, 128, kBits, SB, Y>(x, w, scales, biases, y, M, N, K, group_size, s);
}

template <int kBits, class SB>
int dispatch_y(const void* x, const uint32_t* w, const void* scales, const void* biases, void* y,
               int y_dtype, int M, int N, int K, int group_size, hipStream_t s) {
    if (y_dtype == GDN_F32) return dispatch_qlinear<kBits, SB, ActF32>(x, w, scales, biases, y, M, N, K, group_size, s);
    if (y_dtype == GDN_BF16) return dispatch_qlinear<kBits, SB, ActBF16>(x, w, scales, biases, y, M, N, K, group_size, s);
    return dispatch_qlinear<kBits, SB, ActF16>(x, w, scales, biases, y, M, N, K, group_size, s);
}

template <int kBits>
int dispatch_sb(const void* x, const uint32_t* w, const void* scales, const void* biases, int sb_dtype,
                void* y, int y_dtype, int M, int N, int K, int group_size, hipStream_t s) {
    if (sb_dtype == GDN_F32) return dispatch_y<kBits, ActF32>(x, w, scales, biases, y, y_dtype, M, N, K, group_size, s);
    if (sb_dtype == GDN_BF16) return dispatch_y<kBits, ActBF16>(x, w, scales, biases, y, y_dtype, M, N, K, group_size, s);
    return dispatch_y<kBits, ActF16>(x, w, scales, biases, y, y_dtype, M, N, K, group_size, s);
}

template <int kBits, class SB>
int launch_dequant_out(const uint32_t* w, const void* scales, const void* biases, void* out,
                       int out_dtype, int N, int K, int group_size, hipStream_t s) {
    const int64_t words = int64_t(N) * (K / Packing<kBits>::per_word);
    const dim3 grid(unsigned((words + 255) / 256));
    const auto* sc = static_cast<const typename SB::storage*>(scales);
    const auto* bi = static_cast<const typename SB::storage*>(biases);
    if (out_dtype == GDN_F32)
        hipLaunchKernelGGL((dequantize_kernel<kBits, SB, ActF32>), grid, dim3(256), 0, s, w, sc, bi,
                           static_cast<float*>(out), N, K, group_size);
    else if (out_dtype == GDN_BF16)
        hipLaunchKernelGGL((dequantize_kernel<kBits, SB, ActBF16>), grid, dim3(256), 0, s, w, sc, bi,
                           static_cast<uint16_t*>(out), N, K, group_size);
    else
        hipLaunchKernelGGL((dequantize_kernel<kBits, SB, ActF16>), grid, dim3(256), 0, s, w, sc, bi,
                           static_cast<uint16_t*>(out), N, K, group_size);
    return check_launch("gdn_dequantize");
}

template <int kBits>
int launch_dequant(const uint32_t* w, const void* scales, const void* biases, int sb_dtype, void* out,
                   int out_dtype, int N, int K, int group_size, hipStream_t s) {
    if (sb_dtype == GDN_F32) return launch_dequant_out<kBits, ActF32>(w, scales, biases, out, out_dtype, N, K, group_size, s);
    if (sb_dtype == GDN_BF16) return launch_dequant_out<kBits, ActBF16>(w, scales, biases, out, out_dtype, N, K, group_size, s);
    return launch_dequant_out<kBits, ActF16>(w, scales, biases, out, out_dtype, N, K, group_size, s);
}

int check_quant_args(const char* fn, const void* w, const void* scales, const void* biases,
                     int sb_dtype, int N, int K, int bits, int group_size) {
    GDN_REQUIRE(w && scales && biases, "%s: null weight, scales or biases", fn);
    GDN_REQUIRE(N > 0 && K > 0, "%s: bad sizes N=%d K=%d", fn, N, K);
    GDN_REQUIRE(valid_dtype(sb_dtype), "%s: bad scales/biases dtype", fn);
    if (bits != 4 && bits != 8)
        return fail(GDN_EUNSUPPORTED, "%s: %d-bit weights (4 and 8 are implemented)", fn, bits);
    GDN_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
                "%s: group_size must be 32, 64 or 128 (got %d)", fn, group_size);
    GDN_REQUIRE(K % kBK == 0 && K % group_size == 0, "%s: K=%d must be a multiple of 64 and of group_size", fn, K);
    GDN_REQUIRE(reinterpret_cast<uintptr_t>(w) % 16 == 0, "%s: weight must be 16-byte aligned", fn);
    return 0;
}

}  // namespace
}  // namespace gdn

using namespace gdn;

extern "C" int gdn_quantized_matmul(const void* x, int x_dtype, const void* w, const void* scales,
                                    const void* biases, int sb_dtype, void* y, int y_dtype, int M,
                                    int N, int K, int bits, int group_size, void* stream) {
    if (int rc = check_quant_args("gdn_quantized_matmul", w, scales, biases, sb_dtype, N, K, bits,
                                  group_size))
        return rc;
    GDN_REQUIRE(M >= 0, "gdn_quantized_matmul: bad M=%d", M);
    GDN_REQUIRE(valid_dtype(x_dtype) && valid_dtype(y_dtype), "gdn_quantized_matmul: bad dtype");
    if (x_dtype != GDN_BF16)
        return fail(GDN_EUNSUPPORTED, "gdn_quantized_matmul: x must be bfloat16 (use gdn_dequantize)");
    if (M == 0) return 0;
    GDN_REQUIRE(x && y, "gdn_quantized_matmul: null x or y");
    GDN_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0, "gdn_quantized_matmul: x must be 16-byte aligned");
    GDN_REQUIRE(!overlaps(x, int64_t(M) * K * 2, y, int64_t(M) * N * dtype_size(y_dtype)),
                "gdn_quantized_matmul: y overlaps x");
    hipStream_t s = as_stream(stream);
    const auto* wp = static_cast<const uint32_t*>(w);
    if (bits == 4) return dispatch_sb<4>(x, wp, scales, biases, sb_dtype, y, y_dtype, M, N, K, group_size, s);
    return dispatch_sb<8>(x, wp, scales, biases, sb_dtype, y, y_dtype, M, N, K, group_size, s);
}

extern "C" int gdn_dequantize(const void* w, const void* scales, const void* biases, int sb_dtype,
                              void* out, int out_dtype, int N, int K, int bits, int group_size,
                              void* stream) {
    if (int rc = check_quant_args("gdn_dequantize", w, scales, biases, sb_dtype, N, K, bits, group_size))
        return rc;
    GDN_REQUIRE(out && valid_dtype(out_dtype), "gdn_dequantize: bad output");
    hipStream_t s = as_stream(stream);
    const auto* wp = static_cast<const uint32_t*>(w);
    if (bits == 4) return launch_dequant<4>(wp, scales, biases, sb_dtype, out, out_dtype, N, K, group_size, s);
    return launch_dequant<8>(wp, scales, biases, sb_dtype, out, out_dtype, N, K, group_size, s);
}
