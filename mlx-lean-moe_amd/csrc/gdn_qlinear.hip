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
#include <mutex>
#include <type_traits>

#include "gdn_common.h"
#include "gdn_host.h"

namespace gdn {
namespace {

constexpr int kBK = 64;          // K per pipeline step
constexpr int kTS = kBK + 8;     // bf16 row stride of the LDS tiles

GDN_DEV f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// y[i] with the residual: the product rounded to y's dtype plus residual[i]
// (the unfused add of two y-dtype arrays; the store rounds the sum).
GDN_DEV float plus_residual(float v, const void* residual, int64_t i, int dtype) {
    return residual ? round_to(v, dtype) + load_any(residual, i, dtype) : v;
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
    typename Y::storage* y, const void* residual, int M, int N, int K, int group_size) {
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
                if (m < M && n < N) {
                    const int64_t e = int64_t(m) * N + n;
                    Y::store(y, e, plus_residual(acc[a][b][i], residual, e, Y::code));
                }
            }
        }
}

// Decode-sized M (<= 64): one 512-thread workgroup per kCols (32 or 64)
// output columns over the whole K. The MFMAs take the integer codes, not dequantized
// weights: a wave's k slice of a step (kSlice = 32 or 64 k) lies in one
// quantization group g, so with P = sum_{k in slice} x[m][k] q[n][k] and
// X = sum_{k in slice} x[m][k],
//     y[m][n] = sum over slices of s[n][g] P + b[n][g] X,
// accumulated in float (MLX's matrix-vector kernels apply scale and bias to
// per-group float partial sums in the same way). 4-bit B fragments are the
// bf16 values 1 + q / 16, written straight into bf16 bits two codes per
// bit-and (exact; pairs codes i and i + 4 of a word, so the x tile is staged
// with the matching order of each 8-element chunk), giving
// P' = X + P / 16 and y += 16 s P' + (b - 16 s) X; 8-bit codes convert to
// bf16 exactly (P' = P). X comes from one MFMA against ones.
//
// Every thread first requests its pieces of the workgroup's scales and
// biases, the first step of x and its share of the packed weights for ALL
// steps (16-byte runs of one column), so the HBM stream is in flight at
// once. Each step stages x (16 kMT rows, clamped to M) and the step's
// packed words in LDS; wave w takes k slice [kSlice w, kSlice (w + 1)) of
// the step for the whole 16 kMT x kCols block. The 8 waves' float partial
// blocks are summed in LDS in a fixed order at the end. Needs K a multiple
// of 8 kSlice (kSteps steps), K / group_size <= kDecGroups and a multiple of
// the 16-byte piece's entry count, and 16-byte aligned operands.
//
// kDirect (4-bit codes, 64-k slices, 2 or 4 steps): the codes skip the
// LDS. Wave w takes the contiguous k range [64 kSteps w, 64 kSteps (w + 1))
// of the workgroup's range (its slice of step s is the range's s-th 64 k),
// so each column's codes for a wave are one run of 32 kSteps bytes: lane
// (column c = l % 16, quarter q = l / 16) loads 16-byte piece 4 i + q of
// that run (instruction i of each 16-column tile, all at the start). A
// piece holds 32 codes, four 8-code dwords: the lower half-wave's pieces
// belong to step 2 i, the upper's to step 2 i + 1, and one
// v_permlane32_swap of dwords kb and 2 + kb gives both steps' fragment kb.
// Lane quarter q then holds the slice's k 32 (q & 1) + 16 (q >> 1) + 8 kb
// .. +7 (the x fragments are read in the same order), and the x tile of a
// step gathers the 8 waves' slices. Freed of the weight tile, the LDS holds
// two x tiles at 64 rows: one barrier a step, and the next step's x is
// staged while the other waves compute.
//
// Split K: with gridDim.y = S > 1, workgroup (t, j) takes the k range
// [j K / S, (j + 1) K / S) of column tile t (kSteps steps of it) and stores
// its float32 block at partial[j][M][N]; qlinear_split_sum_kernel adds the
// S blocks in order. It spreads few column tiles (a projection with small
// N) over the CUs.
constexpr int kDecGroups = 64;  // scale groups per column the LDS holds

// The two constants of the 4-bit code fragment, held in registers so that
// each dword is a shift and one v_and_or_b32 (gfx9 VOP3 takes no literals).
struct CodeConsts {
    uint32_t mask, one;
};

GDN_DEV CodeConsts code_consts() {
    CodeConsts k;
    asm volatile("s_mov_b32 %0, 0x780078" : "=s"(k.mask));
    asm volatile("v_mov_b32 %0, 0x3f803f80" : "=v"(k.one));
    return k;
}

template <int kBits>
GDN_DEV bf16x8 code_fragment(const uint32_t* words, CodeConsts k) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 d;
    if constexpr (kBits == 4) {
        // dword i = (1 + q_i / 16, 1 + q_{i+4} / 16): code bits to bf16 mantissa bits 3..6
        const uint32_t q = words[0];
        d[0] = ((q << 3) & k.mask) | k.one;
        d[1] = ((q >> 1) & k.mask) | k.one;
        d[2] = ((q >> 5) & k.mask) | k.one;
        d[3] = ((q >> 9) & k.mask) | k.one;
        return __builtin_bit_cast(bf16x8, d);
    } else {
        bf16x8 b;
        const uint32_t q0 = words[0], q1 = words[1];
#pragma unroll
        for (int j = 0; j < 8; ++j) b[j] = static_cast<__bf16>(float(((j < 4 ? q0 : q1) >> (8 * (j & 3))) & 255u));
        return b;
    }
}

template <int kBits, int kSteps, int kMT, int kSlice, int kCols, bool kXF32, bool kDirect = false>
__global__ __launch_bounds__(512) void qlinear_decode_kernel(
    const void* __restrict__ x_all, const uint32_t* __restrict__ w, const void* __restrict__ scales,
    const void* __restrict__ biases, int sb_dtype, void* y_all, int y_dtype, const void* residual_all, int M_all,
    int N, int K, int group_size, float* __restrict__ partial) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    // Row blocks: workgroup (t, j, z) takes rows [16 kMT z, 16 kMT (z + 1))
    // of x, y and the residual (gridDim.z = 1: all M rows).
    const int row0 = int(blockIdx.z) * 16 * kMT;
    const int M = gridDim.z > 1 ? (M_all - row0 < 16 * kMT ? M_all - row0 : 16 * kMT) : M_all;
    const void* xp = static_cast<const char*>(x_all) + int64_t(row0) * K * (kXF32 ? 4 : 2);
    const int esy = y_dtype == GDN_F32 ? 4 : 2;
    void* y = static_cast<char*>(y_all) + int64_t(row0) * N * esy;
    const void* residual = residual_all ? static_cast<const char*>(residual_all) + int64_t(row0) * N * esy : nullptr;
    constexpr int kStep = 8 * kSlice;            // k per step
    constexpr int kKB = kSlice / 32;             // MFMA k blocks per wave per step
    constexpr int kRows = 16 * kMT;
    constexpr int kTN = kCols / 16;              // 16-column tiles
    constexpr int kXS = kStep + 8;               // bf16 row stride of the x tile
    constexpr int kWPC = kStep * kBits / 32;     // packed words of one column per step
    constexpr int kWS = kWPC + 4;                // word row stride of the weight tile
    constexpr int kXLoads = kRows * kStep / 8 / 512;   // 8-element x chunks per thread per step
    constexpr int kWLoads = kDirect ? 1 : kCols * kWPC / 4 / 512;  // 16-byte weight pieces per thread per step
    static_assert(!kDirect || (kBits == 4 && kSlice == 64 && (kSteps == 2 || kSteps == 4)),
                  "direct code fragments: 4-bit codes, 64-k slices, 2 or 4 steps");
    // first k of wave wv's slice of step s, in the workgroup's range
    auto slice_k = [](int wv_, int s_) { return kDirect ? kSlice * (wv_ * kSteps + s_) : kStep * s_ + kSlice * wv_; };
    // float32 x is staged as two bf16 tiles, hi = bf16(x) and lo =
    // bf16(x - hi) (together x to ~16 significant bits), each fragment
    // taking two MFMAs into the same accumulator
    constexpr int kXParts = kXF32 ? 2 : 1;
    constexpr int kXBytes = kXParts * kRows * kXS * 2;
    constexpr int kWBytes = kDirect ? 0 : kCols * kWS * 4;
    constexpr int kPBytes = 4 * kMT * kTN * 64 * 16;  // 4 partial blocks of kMT x kTN tiles of float4 per lane
    // a group spans at least one slice, so the k range holds at most
    // 8 kSteps groups (and at most kDecGroups, the host's limit)
    constexpr int kGroups = 8 * kSteps < kDecGroups ? 8 * kSteps : kDecGroups;
    constexpr int kSBRow = kCols * (kGroups + 1);
    constexpr int kSBBytes = 2 * kSBRow * 4;
    // double-buffered tiles (one barrier per step) where the LDS holds them,
    // for two workgroups per CU with 32 columns
    constexpr int kBudget = kCols == 32 ? 80 * 1024 : 160 * 1024;
    constexpr int kBufs = 2 * (kXBytes + kWBytes) + kSBBytes <= kBudget ? 2 : 1;
    static_assert(!kDirect || kBufs == 2, "direct code fragments are for double-buffered x tiles");
    constexpr int kMain = kBufs * (kXBytes + kWBytes) > kPBytes ? kBufs * (kXBytes + kWBytes) : kPBytes;
    constexpr int kBQ = (kSteps + 3) / 4;        // bias MFMAs (four of a wave's slices each) per tile
    static_assert(kXLoads >= 1 && kWLoads >= 1, "step too small for 512 threads");
    __shared__ __attribute__((aligned(16))) unsigned char lds[kMain];
    __shared__ float sbs[2 * kSBRow];
    auto xs = [&](int buf) { return reinterpret_cast<uint16_t*>(lds + buf * kXBytes); };  // [kXParts][kRows][kXS]
    auto ws = [&](int buf) { return reinterpret_cast<uint32_t*>(lds + kBufs * kXBytes + buf * kWBytes); };  // [kCols][kWS]
    f32x4* part = reinterpret_cast<f32x4*>(lds);  // [4][kMT][kTN][64] after the steps

    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, lr = l & 15, lq = l >> 4;
    const int n0 = blockIdx.x * kCols;
    const int gpr = K / group_size;
    // this workgroup's k range: split blockIdx.y, kSteps steps from k0, whose
    // gl groups start at group split gl of each column
    const int split = blockIdx.y, k0 = split * kSteps * kStep, gl = kSteps * kStep / group_size;

    // Operands are read with buffer loads: a 32-bit per-thread offset that
    // stays fixed over the steps (rows clamped to M - 1, columns to N - 1;
    // their outputs are not stored) plus a uniform offset in an SGPR.
    // Sizes below 2^31 bytes are checked by the host.
    constexpr int kRaw = 0x00020000;  // buffer resource word 3 of a raw buffer
    const int esx = kXF32 ? 4 : 2, esz = sb_dtype == GDN_F32 ? 4 : 2;
    const int wpr4 = K * kBits / 8;  // bytes of one weight row
    const auto xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(xp), 0, M * K * esx, kRaw);
    const auto wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(w), 0, N * wpr4, kRaw);
    const auto sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(scales), 0, N * gpr * esz, kRaw);
    const auto br = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(biases), 0, N * gpr * esz, kRaw);

    // Scales and biases of the range's groups of the kCols columns, in
    // 16-byte pieces (a piece holds groups of one column): piece p of either
    // array is piece p % ppc of column p / ppc; thread t takes pieces t and
    // t + 512 of both (ppc and per_piece are powers of two).
    const int per_piece = 16 / esz, ppc = gl / per_piece, ppc_shift = __builtin_ctz(ppc);
    const int span_pieces = kCols * ppc;
    u32x4 sv[2], bv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = tid + 512 * i;
        if (p < span_pieces) {
            const int c = p >> ppc_shift, pc = p & (ppc - 1);
            const int col = n0 + c < N ? n0 + c : N - 1;
            const int off = col * gpr * esz + 16 * pc, soff = split * gl * esz;
            sv[i] = __builtin_amdgcn_raw_buffer_load_b128(sr, off, soff, 0);
            bv[i] = __builtin_amdgcn_raw_buffer_load_b128(br, off, soff, 0);
        }
    }

    constexpr int kChunksPerRow = kStep / 8, kXRowStep = 512 / kChunksPerRow;
    typedef float f32x8 __attribute__((ext_vector_type(8)));
    using xchunk_t = std::conditional_t<kXF32, f32x8, u16x8>;
    int xoffs[kXLoads];
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
        const int r = tid / kChunksPerRow + i * kXRowStep;
        // chunk ch of a step's tile: 8 k of wave ch / 8's slice (kDirect), or
        // of the step's contiguous k
        const int ch = tid % kChunksPerRow;
        const int kc = kDirect ? (ch >> 3) * kSteps * kSlice + 8 * (ch & 7) : 8 * ch;
        xoffs[i] = ((r < M ? r : M - 1) * K + kc) * esx;
    }
    xchunk_t xv[kXLoads];
    auto fetch_x = [&](int s) {
        const int soff = (k0 + (kDirect ? kSlice : kStep) * s) * esx;
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int o = xoffs[i];
            if constexpr (kXF32) {
                const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(xr, o, soff, 0);
                const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(xr, o + 16, soff, 0);
                xv[i] = __builtin_bit_cast(f32x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            } else {
                xv[i] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(xr, o, soff, 0));
            }
        }
    };
    // 4-bit fragments pair codes i and i + 4 of a word: stage each chunk in
    // that order
    auto order = [&](u16x8 v) {
        if constexpr (kBits == 4) return u16x8(__builtin_shufflevector(v, v, 0, 4, 1, 5, 2, 6, 3, 7));
        else return v;
    };
    auto stage_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int r = tid / kChunksPerRow + i * kXRowStep, ch = tid % kChunksPerRow;
            uint16_t* dst = &xs(buf)[r * kXS + 8 * ch];
            if constexpr (kXF32) {
                bf16x8 hi, lo;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    hi[j] = static_cast<__bf16>(xv[i][j]);
                    lo[j] = static_cast<__bf16>(xv[i][j] - static_cast<float>(hi[j]));
                }
                *reinterpret_cast<u16x8*>(dst) = order(__builtin_bit_cast(u16x8, hi));
                *reinterpret_cast<u16x8*>(dst + kRows * kXS) = order(__builtin_bit_cast(u16x8, lo));
            } else {
                *reinterpret_cast<u16x8*>(dst) = order(xv[i]);
            }
        }
    };
    fetch_x(0);

    // kDirect: the wave's code pieces for every step, requested now
    // (instruction i of tile tn: piece 4 i + lq of column 16 tn + lr)
    u32x4 wd[kDirect ? kSteps / 2 : 1][kTN];
    if constexpr (kDirect) {
#pragma unroll
        for (int tn = 0; tn < kTN; ++tn) {
            const int col = n0 + 16 * tn + lr;
            const int o = (col < N ? col : N - 1) * wpr4 + slice_k(wv, 0) / 2 + 16 * lq;
#pragma unroll
            for (int i = 0; i < kSteps / 2; ++i)
                wd[i][tn] = __builtin_amdgcn_raw_buffer_load_b128(wr, o + 64 * i, k0 / 2, 0);
        }
    }
    // packed weights of every step: piece i of a step is 16-byte piece wpc of
    // column wc0 + i kWColStep (clamped)
    constexpr int kPiecesPerCol = kWPC / 4, kWColStep = 512 / kPiecesPerCol;
    const int wc0 = tid / kPiecesPerCol, wpc = tid % kPiecesPerCol;
    int woff[kWLoads];
#pragma unroll
    for (int i = 0; i < kWLoads; ++i) {
        const int col = n0 + wc0 + i * kWColStep;
        woff[i] = (col < N ? col : N - 1) * wpr4 + 16 * wpc;
    }
    // the first kPre steps' pieces are requested now (all of them where 32
    // registers hold them; 16 for the 16-step kernels, whose unrolled loop
    // holds more), each later step's when its slot is staged
    constexpr int kWRegPieces = kSteps >= 16 ? 4 : 8;
    constexpr int kPre = kWRegPieces / kWLoads < kSteps ? (kWRegPieces / kWLoads > 0 ? kWRegPieces / kWLoads : 1) : kSteps;
    u32x4 wq[kPre][kWLoads];
    auto load_w = [&](int s) {
#pragma unroll
        for (int i = 0; i < kWLoads; ++i)
            wq[s % kPre][i] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff[i], (k0 * kBits / 8) + 4 * kWPC * s, 0);
    };
    if constexpr (!kDirect) {
#pragma unroll
        for (int s = 0; s < kPre; ++s) load_w(s);
    }
    auto stage_w = [&](int buf, int s) {
        if constexpr (kDirect) return;
#pragma unroll
        for (int i = 0; i < kWLoads; ++i)
            *reinterpret_cast<u32x4*>(&ws(buf)[(wc0 + i * kWColStep) * kWS + 4 * wpc]) = wq[s % kPre][i];
        if (s + kPre < kSteps) load_w(s + kPre);
    };

    // scales and biases to float, [which][column][group] with rows of gl + 1
    auto to_float = [&](u32x4 v, float* d) {
        if (sb_dtype == GDN_F32) {
#pragma unroll
            for (int j = 0; j < 4; ++j) d[j] = __uint_as_float(v[j]);
        } else if (sb_dtype == GDN_BF16) {
#pragma unroll
            for (int j = 0; j < 8; ++j) d[j] = __uint_as_float((j & 1) ? v[j >> 1] & 0xFFFF0000u : v[j >> 1] << 16);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) d[j] = f16_bits_to_f32(uint16_t(v[j >> 1] >> (16 * (j & 1))));
        }
    };
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = tid + 512 * i;
        if (p < span_pieces) {
            const int c = p >> ppc_shift, pc = p & (ppc - 1);
            to_float(sv[i], sbs + c * (gl + 1) + pc * per_piece);
            to_float(bv[i], sbs + kSBRow + c * (gl + 1) + pc * per_piece);
        }
    }

    f32x4 acc[kMT][kTN];
#pragma unroll
    for (int tm = 0; tm < kMT; ++tm)
#pragma unroll
        for (int tn = 0; tn < kTN; ++tn) acc[tm][tn] = f32x4{0.f, 0.f, 0.f, 0.f};
    // xa[q][tm]: the row sum X of row 16 tm + lr over this wave's slice of
    // step 4 q + lq, the A operand of the bias MFMAs
    float xa[kBQ][kMT];
#pragma unroll
    for (int q = 0; q < kBQ; ++q)
#pragma unroll
        for (int tm = 0; tm < kMT; ++tm) xa[q][tm] = 0.f;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    bf16x8 ones;
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = static_cast<__bf16>(1.0f);
    constexpr float kQScale = kBits == 4 ? 16.f : 1.f;  // P = kQScale (P' - X) for 4-bit codes
    const CodeConsts kc = code_consts();

    // wave wv's slice of step s from tile buffer buf: acc += kQScale s P'
    auto compute = [&](int buf, int s) {
        const uint16_t* xb = xs(buf);
        const uint32_t* wb = ws(buf);
        const int g = slice_k(wv, s) / group_size;
        bf16x8 a[kXParts][kMT][kKB];
        if constexpr (kDirect) {
            // steps 2 i and 2 i + 1 of every tile: dwords kb and 2 + kb swapped
            // across the half-waves give fragment kb of both
            if (s % 2 == 0) {
#pragma unroll
                for (int tn = 0; tn < kTN; ++tn)
#pragma unroll
                    for (int kb = 0; kb < kKB; ++kb) {
                        const auto r = __builtin_amdgcn_permlane32_swap(wd[s / 2][tn][kb], wd[s / 2][tn][2 + kb],
                                                                       false, false);
                        wd[s / 2][tn][kb] = r[0];
                        wd[s / 2][tn][2 + kb] = r[1];
                    }
            }
        }
#pragma unroll
        for (int tm = 0; tm < kMT; ++tm) {
            // ones times the x fragment as the B operand: every element of
            // lane (r, *) is the sum of row 16 tm + r over the slice
            f32x4 X = zero;
#pragma unroll
            for (int h = 0; h < kXParts; ++h)
#pragma unroll
                for (int kb = 0; kb < kKB; ++kb) {
                    const int ch = kDirect ? 32 * (lq & 1) + 16 * (lq >> 1) + 8 * kb : 32 * kb + 8 * lq;
                    a[h][tm][kb] = *reinterpret_cast<const bf16x8*>(
                        &xb[(h * kRows + 16 * tm + lr) * kXS + kSlice * wv + ch]);
                    X = mfma_bf16(ones, a[h][tm][kb], X);
                }
            if (lq == (s & 3)) xa[s / 4][tm] = X[0];
        }
#pragma unroll
        for (int tn = 0; tn < kTN; ++tn) {
            const int c = 16 * tn + lr;
            const float sp = kQScale * sbs[c * (gl + 1) + g];
            bf16x8 bq[kKB];
#pragma unroll
            for (int kb = 0; kb < kKB; ++kb) {
                if constexpr (kDirect) {
                    const uint32_t word = wd[s / 2][tn][(s % 2) * 2 + kb];
                    bq[kb] = code_fragment<kBits>(&word, kc);
                } else {
                    bq[kb] = code_fragment<kBits>(&wb[c * kWS + (kSlice * wv + 32 * kb + 8 * lq) * kBits / 32], kc);
                }
            }
#pragma unroll
            for (int tm = 0; tm < kMT; ++tm) {
                f32x4 P = zero;
#pragma unroll
                for (int h = 0; h < kXParts; ++h)
#pragma unroll
                    for (int kb = 0; kb < kKB; ++kb) P = mfma_bf16(a[h][tm][kb], bq[kb], P);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[tm][tn][i] = __builtin_fmaf(sp, P[i], acc[tm][tn][i]);
            }
        }
    };

    if constexpr (kBufs == 2) {
        stage_x(0);
        stage_w(0, 0);
        __syncthreads();
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const int buf = s & 1;
            if (s + 1 < kSteps) fetch_x(s + 1);
            compute(buf, s);
            if (s + 1 < kSteps) {
                stage_x(buf ^ 1);
                stage_w(buf ^ 1, s + 1);
            }
            __syncthreads();
        }
    } else {
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            if (s > 0) __syncthreads();  // the previous step's reads of the tiles are done
            stage_x(0);
            stage_w(0, s);
            __syncthreads();
            if (s + 1 < kSteps) fetch_x(s + 1);
            compute(0, s);
        }
        __syncthreads();
    }

    // The bias terms of the wave's slices: acc += X b' summed over the
    // slices, b' = b - 16 s for 4-bit codes (undoing their 1 + q / 16
    // offset) and b for 8-bit ones,
    // as v_mfma_f32_16x16x4f32 with A[row][j] = X of step 4 q + j and
    // B[j][column] = b' of that step's group (the sbs rows are
    // still intact: only the tile region of the LDS is reused below).
#pragma unroll
    for (int q = 0; q < kBQ; ++q) {
        const int st = 4 * q + lq;
        const int g = slice_k(wv, st) / group_size;
#pragma unroll
        for (int tn = 0; tn < kTN; ++tn) {
            const int c = 16 * tn + lr;
            float bb = 0.f;
            if (st < kSteps) {
                bb = sbs[kSBRow + c * (gl + 1) + g];
                if constexpr (kBits == 4) bb = __builtin_fmaf(-kQScale, sbs[c * (gl + 1) + g], bb);
            }
#pragma unroll
            for (int tm = 0; tm < kMT; ++tm)
                acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[q][tm], bb, acc[tm][tn], 0, 0, 0);
        }
    }

    // Sum of the 8 waves' blocks: waves 4-7 hand theirs to waves 0-3, which
    // add them in place; every thread then adds the 4 sums for its outputs.
    // A block holds each lane's kMT x kTN tiles as float4 at
    // [(blk kMT + tm) kTN + tn][lane].
    f32x4* mine = part + (wv & 3) * kMT * kTN * 64 + l;
    if (wv >= 4) {
#pragma unroll
        for (int tm = 0; tm < kMT; ++tm)
#pragma unroll
            for (int tn = 0; tn < kTN; ++tn) mine[(tm * kTN + tn) * 64] = acc[tm][tn];
    }
    __syncthreads();
    if (wv < 4) {
#pragma unroll
        for (int tm = 0; tm < kMT; ++tm)
#pragma unroll
            for (int tn = 0; tn < kTN; ++tn)
                mine[(tm * kTN + tn) * 64] = acc[tm][tn] + mine[(tm * kTN + tn) * 64];
    }
    __syncthreads();
    // float4 f = tid + 512 j of a block: tile f / 64 = tm kTN + tn, lane f % 64,
    // rows 16 tm + 4 (lane / 16) + i, column 16 tn + lane % 16
    constexpr int kF = kMT * kTN * 64;
    auto store = [&](auto put) {
#pragma unroll
        for (int j = 0; j < (kF + 511) / 512; ++j) {
            const int f = tid + 512 * j;
            if (f < kF) {
                const f32x4 v = (part[f] + part[kF + f]) + (part[2 * kF + f] + part[3 * kF + f]);
                const int t = f >> 6, ln = f & 63, tm = t / kTN, tn = t % kTN;
                const int n = n0 + 16 * tn + (ln & 15), m0 = 16 * tm + 4 * (ln >> 4);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (m0 + i < M && n < N) put(int64_t(m0 + i) * N + n, v[i]);
            }
        }
    };
    if (partial) {
        float* pp = partial + int64_t(split) * M * N;
        store([&](int64_t i, float v) { pp[i] = v; });
    } else if (y_dtype == GDN_BF16)
        store([&](int64_t i, float v) {
            static_cast<uint16_t*>(y)[i] = f32_to_bf16_bits(plus_residual(v, residual, i, GDN_BF16));
        });
    else if (y_dtype == GDN_F16)
        store([&](int64_t i, float v) {
            static_cast<uint16_t*>(y)[i] = f32_to_f16_bits(plus_residual(v, residual, i, GDN_F16));
        });
    else
        store([&](int64_t i, float v) { static_cast<float*>(y)[i] = plus_residual(v, residual, i, GDN_F32); });
}

// y = the sum, in split order, of the split-K kernel's S float32 blocks
// partial[S][count] (plus the residual). A thread takes four consecutive
// elements and requests all 4 S values before the first add (a loop over a
// run-time S waited a memory latency per split: 3.7-4.1 us for the layer's
// out_proj at 64 rows).
template <int S>
__global__ __launch_bounds__(256) void qlinear_split_sum_kernel(const float* __restrict__ partial, int64_t count,
                                                                void* y, int y_dtype, const void* residual) {
    const int64_t i0 = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i0 >= count) return;
    if ((count & 3) == 0) {  // whole float4s: partial is 16-byte aligned
        float4 p[S];
#pragma unroll
        for (int j = 0; j < S; ++j) p[j] = *reinterpret_cast<const float4*>(partial + j * count + i0);
        float4 v = p[0];
#pragma unroll
        for (int j = 1; j < S; ++j) {
            v.x += p[j].x;
            v.y += p[j].y;
            v.z += p[j].z;
            v.w += p[j].w;
        }
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) store_any(y, i0 + e, y_dtype, plus_residual(vv[e], residual, i0 + e, y_dtype));
    } else {
        for (int64_t i = i0; i < i0 + 4 && i < count; ++i) {
            float p[S];
#pragma unroll
            for (int j = 0; j < S; ++j) p[j] = partial[j * count + i];
            float v = p[0];
#pragma unroll
            for (int j = 1; j < S; ++j) v += p[j];
            store_any(y, i, y_dtype, plus_residual(v, residual, i, y_dtype));
        }
    }
}

// The split sum for S = 2, 4, 8 or 16 blocks (the split counts the split-K
// kernels choose).
int launch_split_sum(const float* partial, int splits, int64_t count, void* y, int y_dtype, const void* residual,
                     hipStream_t s, const char* who) {
    const dim3 grid(unsigned(((count + 3) / 4 + 255) / 256));
    switch (splits) {
        case 2: hipLaunchKernelGGL(qlinear_split_sum_kernel<2>, grid, dim3(256), 0, s, partial, count, y, y_dtype, residual); break;
        case 4: hipLaunchKernelGGL(qlinear_split_sum_kernel<4>, grid, dim3(256), 0, s, partial, count, y, y_dtype, residual); break;
        case 8: hipLaunchKernelGGL(qlinear_split_sum_kernel<8>, grid, dim3(256), 0, s, partial, count, y, y_dtype, residual); break;
        case 16: hipLaunchKernelGGL(qlinear_split_sum_kernel<16>, grid, dim3(256), 0, s, partial, count, y, y_dtype, residual); break;
        default: return fail(GDN_EINVAL, "%s: %d splits (2, 4, 8 or 16)", who, splits);
    }
    return check_launch(who);
}

constexpr int kCUs = 256;  // compute units of an MI355X

// Split count for `tiles` column tiles of `ks` steps: the largest power of
// two S <= 16 dividing ks whose k ranges hold whole 16-byte scale pieces of
// each column, with at most one workgroup per CU (measured: beyond that the
// partial blocks cost more than the extra workgroups gain) and S M N floats
// in the workspace; 1 is no split.
int decode_splits(int tiles, int ks, int K, int group_size, int per_piece, int M, int N, int64_t ws_bytes) {
    int best = 1;
    for (int sp = 2; sp <= 16 && ks % sp == 0; sp *= 2) {
        const int gl = K / sp / group_size;
        if (gl % per_piece != 0 || int64_t(tiles) * sp > kCUs || int64_t(sp) * M * N * 4 > ws_bytes) break;
        best = sp;
    }
    return best;
}

template <int kBits, int kMT, int kSlice, int kCols, bool kXF32>
int launch_decode_mt(const void* x, const uint32_t* w, const void* scales, const void* biases, int sb_dtype,
                     void* y, int y_dtype, const void* residual, int M, int N, int K, int group_size,
                     void* workspace, int64_t ws_bytes, hipStream_t s, int row_blocks = 1) {
    const int tiles = (N + kCols - 1) / kCols, ks = K / (8 * kSlice);
    const int splits = row_blocks > 1 ? 1
                                      : decode_splits(tiles, ks, K, group_size, sb_dtype == GDN_F32 ? 4 : 8, M, N,
                                                      workspace ? ws_bytes : 0);
    float* partial = splits > 1 ? static_cast<float*>(workspace) : nullptr;
    if (partial)
        GDN_REQUIRE(!overlaps(partial, int64_t(splits) * M * N * 4, y, int64_t(M) * N * dtype_size(y_dtype)) &&
                        !overlaps(partial, int64_t(splits) * M * N * 4, x, int64_t(M) * K * (kXF32 ? 4 : 2)),
                    "gdn_quantized_matmul: workspace overlaps x or y");
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(splits), static_cast<unsigned>(row_blocks));
    // 17-64 rows of bf16 x against 4-bit codes in 64-k slices take the code
    // fragments straight from memory (two x tiles in the LDS) at 2 or 4 steps
#define GDN_DEC(STEPS)                                                                                       \
    hipLaunchKernelGGL((qlinear_decode_kernel<kBits, STEPS, kMT, kSlice, kCols, kXF32,                        \
                                              kBits == 4 && kSlice == 64 && kMT >= 2 && !kXF32 &&         \
                                                  (STEPS == 2 || STEPS == 4)>),                           \
                       grid, dim3(512), 0, s, x, w, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K,   \
                       group_size, partial)
    switch (ks / splits) {
        case 1: GDN_DEC(1); break;
        case 2: GDN_DEC(2); break;
        case 4: GDN_DEC(4); break;
        case 8:
            if constexpr (kBits == 4 || kSlice == 32) {
                GDN_DEC(8);
                break;
            }
            return -1;
        case 16:
            if constexpr (kBits == 4 && kSlice == 32) {
                GDN_DEC(16);
                break;
            }
            return -1;
        default: return -1;
    }
#undef GDN_DEC
    if (int rc = check_launch("gdn_quantized_matmul")) return rc;
    if (!partial) return 0;
    return launch_split_sum(partial, splits, int64_t(M) * N, y, y_dtype, residual, s, "gdn_quantized_matmul");
}

// The k slice a wave takes per step: one whole group of 32, else 64 k.
int decode_slice(int group_size) { return group_size == 32 ? 32 : 64; }

// Whether the decode kernel takes this shape (M <= 64 checked by the
// caller): the step counts launch_decode_mt instantiates, the scale rows the
// LDS holds, scales in whole 16-byte pieces of one column.
bool decode_shape_fits(int sb_dtype, int N, int K, int bits, int group_size) {
    const int slice = decode_slice(group_size), step = 8 * slice;
    const int ks = K / step, gpr = K / group_size, per_piece = sb_dtype == GDN_F32 ? 4 : 8;
    const int words_per_thread = ks * step * bits / 32 / 8;  // packed weight words each thread holds
    const bool steps_ok = K % step == 0 && (ks == 1 || ks == 2 || ks == 4 || ks == 8 || ks == 16) &&
                          words_per_thread <= 64;
    // 32-bit buffer offsets: the packed weights under 2^31 bytes
    return steps_ok && gpr <= kDecGroups && gpr % per_piece == 0 && int64_t(N) * K * bits / 8 < (int64_t(1) << 31);
}

// ... and these operands: 16-byte aligned.
bool decode_kernel_fits(const void* x, const uint32_t* w, const void* scales, const void* biases, int sb_dtype,
                        int N, int K, int bits, int group_size) {
    const auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    return decode_shape_fits(sb_dtype, N, K, bits, group_size) && al(x) && al(w) && al(scales) && al(biases);
}

// Columns per decode workgroup (the choice launch_decode makes).
int decode_cols(bool x_f32, int mt, int bits, int group_size) {
    const int narrow = bits == 4 && decode_slice(group_size) == 32 ? 64 : 32;
    return (x_f32 ? mt == 1 : mt <= 2) ? narrow : 64;
}

// Sum over the 64 lanes of a wave, complete in lane 63: pairs and quads
// (quad_perm), then row_shr 4 and 8 (lane 15 of each row holds the row's
// sum), then row_bcast 15 and 31 (DPP lanes with no source add 0).
GDN_DEV float wave_sum_lane63(float v) {
#define GDN_DPP_ADD(CTRL, ROWS) \
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false))
    GDN_DPP_ADD(0xB1, 0xF);   // quad_perm [1, 0, 3, 2]
    GDN_DPP_ADD(0x4E, 0xF);   // quad_perm [2, 3, 0, 1]
    GDN_DPP_ADD(0x114, 0xF);  // row_shr 4
    GDN_DPP_ADD(0x118, 0xF);  // row_shr 8
    GDN_DPP_ADD(0x142, 0xA);  // row_bcast 15 into rows 1 and 3
    GDN_DPP_ADD(0x143, 0xC);  // row_bcast 31 into rows 2 and 3
#undef GDN_DPP_ADD
    return v;
}

// Matrix-vector kernel for kM rows of x (the dispatch uses one) and 4-bit
// codes: one wave per output column at a time, two columns per wave and
// round of the grid. Lane l takes 16 bytes of packed codes of each of kR
// rounds of a weight row (chunk 64 r + l: 32 codes inside one quantization
// group) and holds the matching x in registers for every column it visits.
// Per chunk and row, with P = sum x q and X = sum x over the chunk,
// y += s P + b X, the wave's lanes summed at the end of the column (the
// per-group float scaling of MLX's matrix-vector kernels). bf16 x: q enters
// as the bf16 pair 1 + q / 16 of codes i and i + 4 of a word (one shift and
// one v_and_or_b32 per pair) against x held as the bf16 pairs
// (x[i], x[i + 4]) in v_dot2c_f32_bf16, so P' = X + P / 16 and
// y += 16 s P' + (b - 16 s) X. float32 x: exact float products of the codes
// (byte conversions) and x.
template <int kBits, int kM, int kR, bool kXF32>
__global__ __launch_bounds__(256) void qlinear_gemv_kernel(
    const void* __restrict__ xp, const uint32_t* __restrict__ w, const void* __restrict__ scales,
    const void* __restrict__ biases, int sb_dtype, void* y, int y_dtype, const void* residual, int M, int N,
    int K, int group_size) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    static_assert(kBits == 4, "4-bit codes");
    constexpr int kCodes = 128 / kBits;                  // codes of a lane's 16-byte chunk
    constexpr bool kPairs = kBits == 4 && !kXF32;         // bf16 pairs and v_dot2c
    constexpr int kXRegs = kPairs ? kCodes / 2 : kCodes;  // x registers per row and round
    constexpr int kRaw = 0x00020000;
    const int lane = threadIdx.x & 63;
    const int wave = int(blockIdx.x) * 4 + int(threadIdx.x >> 6), waves = int(gridDim.x) * 4;
    const int gpr = K / group_size, wpr4 = K * kBits / 8;
    const int esx = kXF32 ? 4 : 2, esz = sb_dtype == GDN_F32 ? 4 : 2;
    const auto wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(w), 0, N * wpr4, kRaw);
    const auto xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(xp), 0, M * K * esx, kRaw);
    const auto sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(scales), 0, N * gpr * esz, kRaw);
    const auto br = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(biases), 0, N * gpr * esz, kRaw);

    // this lane's chunks: k0 = kCodes (64 r + lane), active below K
    bool active[kR];
    int grp[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
        const int k0 = kCodes * (64 * r + lane);
        active[r] = k0 < K;
        grp[r] = active[r] ? k0 / group_size : 0;
    }
    // columns kC (wave + i waves) + c, c < kC: the loads of a wave's kC
    // columns are issued together (the first batch's before x is read), and
    // the other waves of the SIMD cover their latency
    constexpr int kC = 2;
    u32x4 cq[kC][kR];
    uint32_t cs[kC][kR], cb[kC][kR];
    const int esz4 = esz;
    auto fetch = [&](int n0) {
#pragma unroll
        for (int c = 0; c < kC; ++c)
#pragma unroll
            for (int r = 0; r < kR; ++r) {
                const int n = n0 + c;
                cq[c][r] = u32x4{0u, 0u, 0u, 0u};
                cs[c][r] = cb[c][r] = 0u;
                if (active[r] && n < N) {
                    cq[c][r] = __builtin_amdgcn_raw_buffer_load_b128(wr, n * wpr4 + 16 * (64 * r + lane), 0, 0);
                    const int so = (n * gpr + grp[r]) * esz4;
                    if (esz4 == 4) {
                        cs[c][r] = __builtin_amdgcn_raw_buffer_load_b32(sr, so, 0, 0);
                        cb[c][r] = __builtin_amdgcn_raw_buffer_load_b32(br, so, 0, 0);
                    } else {
                        cs[c][r] = __builtin_amdgcn_raw_buffer_load_b16(sr, so, 0, 0);
                        cb[c][r] = __builtin_amdgcn_raw_buffer_load_b16(br, so, 0, 0);
                    }
                }
            }
    };
    int n0 = kC * wave;
    if (n0 < N) fetch(n0);

    // x of the chunks and their sums; rows >= M and inactive chunks hold 0
    uint32_t xq[kM][kR][kXRegs];
    float xs[kM][kR];
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            float v[kCodes];
#pragma unroll
            for (int j = 0; j < kCodes; ++j) v[j] = 0.f;
            if (m < M && active[r]) {
                const int off = (m * K + kCodes * (64 * r + lane)) * esx;
#pragma unroll
                for (int c = 0; c < kCodes * esx / 16; ++c) {
                    const u32x4 d = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16 * c, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (kXF32) {
                            v[4 * c + e] = __uint_as_float(d[e]);
                        } else {
                            v[8 * c + 2 * e] = __uint_as_float(d[e] << 16);
                            v[8 * c + 2 * e + 1] = __uint_as_float(d[e] & 0xFFFF0000u);
                        }
                    }
                }
            }
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < kCodes; ++j) sum += v[j];
            xs[m][r] = sum;
            if constexpr (kPairs) {
                // dword 4 t + i: (x[8 t + i], x[8 t + i + 4]) as bf16 (exact: x is bf16)
#pragma unroll
                for (int t = 0; t < kCodes / 8; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        xq[m][r][4 * t + i] = (__float_as_uint(v[8 * t + i]) >> 16) |
                                              (__float_as_uint(v[8 * t + i + 4]) & 0xFFFF0000u);
            } else {
#pragma unroll
                for (int j = 0; j < kCodes; ++j) xq[m][r][j] = __float_as_uint(v[j]);
            }
        }

    auto sb_value = [&](uint32_t raw) {
        if (sb_dtype == GDN_F32) return __uint_as_float(raw);
        if (sb_dtype == GDN_BF16) return __uint_as_float(raw << 16);
        return f16_bits_to_f32(uint16_t(raw));
    };
    const CodeConsts kc = code_consts();
    // byte j of v as a float (one v_cvt_f32_ubyte<j>)
    auto ubyte = [](uint32_t v, int j) { return float((v >> (8 * j)) & 0xFFu); };

    for (; n0 < N; n0 += kC * waves) {
#pragma unroll
        for (int c = 0; c < kC; ++c) {
            const int n = n0 + c;
            float acc[kM];
#pragma unroll
            for (int m = 0; m < kM; ++m) acc[m] = 0.f;
#pragma unroll
            for (int r = 0; r < kR; ++r) {
                const float s = sb_value(cs[c][r]), b = sb_value(cb[c][r]);
                float P[kM];
#pragma unroll
                for (int m = 0; m < kM; ++m) P[m] = 0.f;
#pragma unroll
                for (int t = 0; t < 4; ++t) {  // the chunk's four words
                    const uint32_t q = cq[c][r][t];
                    if constexpr (kPairs) {
                        // the code_fragment dwords, as scalars (a bit cast of a
                        // vector element reads element 0 on this compiler)
                        const uint32_t d[4] = {((q << 3) & kc.mask) | kc.one, ((q >> 1) & kc.mask) | kc.one,
                                               ((q >> 5) & kc.mask) | kc.one, ((q >> 9) & kc.mask) | kc.one};
#pragma unroll
                        for (int i = 0; i < 4; ++i)
#pragma unroll
                            for (int m = 0; m < kM; ++m)
                                P[m] = __builtin_amdgcn_fdot2_f32_bf16(
                                    __builtin_bit_cast(bf16x2, d[i]), __builtin_bit_cast(bf16x2, xq[m][r][4 * t + i]),
                                    P[m], false);
                    } else {
                        // even codes in the bytes of e, odd ones in those of o
                        const uint32_t e = q & 0x0F0F0F0Fu, o = (q >> 4) & 0x0F0F0F0Fu;
                        const float qv[8] = {ubyte(e, 0), ubyte(o, 0), ubyte(e, 1), ubyte(o, 1),
                                             ubyte(e, 2), ubyte(o, 2), ubyte(e, 3), ubyte(o, 3)};
#pragma unroll
                        for (int j = 0; j < 8; ++j)
#pragma unroll
                            for (int m = 0; m < kM; ++m)
                                P[m] = __builtin_fmaf(__uint_as_float(xq[m][r][8 * t + j]), qv[j], P[m]);
                    }
                }
#pragma unroll
                for (int m = 0; m < kM; ++m) {
                    if constexpr (kPairs)
                        acc[m] += __builtin_fmaf(16.f * s, P[m], __builtin_fmaf(-16.f, s, b) * xs[m][r]);
                    else
                        acc[m] += __builtin_fmaf(s, P[m], b * xs[m][r]);
                }
            }
            // the column's sum over the wave's lanes, in lane 63
#pragma unroll
            for (int m = 0; m < kM; ++m) acc[m] = wave_sum_lane63(acc[m]);
            if (lane == 63 && n < N) {
#pragma unroll
                for (int m = 0; m < kM; ++m)
                    if (m < M) {
                        const int64_t e = int64_t(m) * N + n;
                        store_any(y, e, y_dtype, plus_residual(acc[m], residual, e, y_dtype));
                    }
            }
        }
        if (n0 + kC * waves < N) fetch(n0 + kC * waves);
    }
}

// Rounds of 64 lane chunks a row needs, or 0 where the matrix-vector kernel
// does not take the call. It runs one row of 4-bit codes (K up to 4096,
// all the decode kernel takes at this width): measured against the decode
// kernel at N=12352, K=2048 it takes 6.4 vs 8.3 us (bf16 x) and 10.3 vs
// 10.7 us (float32 x), at N=2048, K=4096 4.8 vs 6.8 us; from two rows on,
// and for 8-bit codes, the decode kernel was as fast or faster.
int gemv_rounds(bool, int M, int K, int bits) {
    if (M != 1 || bits != 4) return 0;
    const int chunk_k = 64 * 32;
    const int r = (K + chunk_k - 1) / chunk_k;
    return r <= 1 ? 1 : r <= 2 ? 2 : 0;
}

template <int kBits, int kM, int kR, bool kXF32>
int launch_gemv_t(const void* x, const uint32_t* w, const void* scales, const void* biases, int sb_dtype, void* y,
                  int y_dtype, const void* residual, int M, int N, int K, int group_size, hipStream_t s) {
    const int waves = (N + 1) / 2 < 16384 ? (N + 1) / 2 : 16384;  // two columns a wave
    hipLaunchKernelGGL((qlinear_gemv_kernel<kBits, kM, kR, kXF32>), dim3(unsigned((waves + 3) / 4)), dim3(256), 0, s,
                       x, w, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, group_size);
    return check_launch("gdn_quantized_matmul");
}

int launch_gemv(const void* x, bool x_f32, const uint32_t* w, const void* scales, const void* biases, int sb_dtype,
                void* y, int y_dtype, const void* residual, int M, int N, int K, int, int group_size, int rounds,
                hipStream_t s) {
#define GDN_GEMV(R, XF32) \
    return launch_gemv_t<4, 1, R, XF32>(x, w, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, group_size, s)
    if (rounds == 1) {
        if (x_f32) GDN_GEMV(1, true);
        GDN_GEMV(1, false);
    }
    if (x_f32) GDN_GEMV(2, true);
    GDN_GEMV(2, false);
#undef GDN_GEMV
}

// Up to 32 rows, workgroups of 32 columns where every thread still gets a
// weight piece (64-k slices or 8-bit codes): two fit on a CU, which doubles
// the waves that hide the LDS and MFMA latencies and spreads the columns
// over all CUs. 33-64 rows keep 64 columns (the LDS holds one workgroup).
// float32 x (twice the x tiles) runs up to 32 rows: 32 columns up to 16
// rows, 64 beyond.
// 17-64 rows of bf16 x against 4-bit codes in 64-k slices, for a
// projection with few column tiles (the layer's out_proj): 16-row blocks of
// the 16-row kernel (grid z), all in one launch, with no split of K.
int decode_row_blocks(bool x_f32, int M, int N, int bits, int group_size) {
    if (x_f32 || M <= 16 || bits != 4 || decode_slice(group_size) != 64) return 1;
    const int rb = (M + 15) / 16, tiles = (N + 31) / 32;
    return (N + 63) / 64 < 128 && int64_t(tiles) * rb <= kCUs ? rb : 1;
}

int launch_decode(const void* x, bool x_f32, const uint32_t* w, const void* scales, const void* biases,
                  int sb_dtype, void* y, int y_dtype, const void* residual, int M, int N, int K, int bits,
                  int group_size, void* workspace, int64_t ws_bytes, hipStream_t s) {
    const int mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
#define GDN_ARGS x, w, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, group_size, workspace, ws_bytes, s
    if (const int rb = decode_row_blocks(x_f32, M, N, bits, group_size); rb > 1)
        return launch_decode_mt<4, 1, 64, 32, false>(GDN_ARGS, rb);
#define GDN_MT(BITS, SLICE, NARROW)                                                       \
    do {                                                                                  \
        if (x_f32) {                                                                      \
            if (mt == 1) return launch_decode_mt<BITS, 1, SLICE, NARROW, true>(GDN_ARGS); \
            return launch_decode_mt<BITS, 2, SLICE, 64, true>(GDN_ARGS);                  \
        }                                                                                 \
        if (mt == 1) return launch_decode_mt<BITS, 1, SLICE, NARROW, false>(GDN_ARGS);    \
        if (mt == 2) return launch_decode_mt<BITS, 2, SLICE, NARROW, false>(GDN_ARGS);    \
        return launch_decode_mt<BITS, 4, SLICE, 64, false>(GDN_ARGS);                     \
    } while (0)
    if (bits == 4) {
        if (decode_slice(group_size) == 32) GDN_MT(4, 32, 64);
        GDN_MT(4, 64, 32);
    }
    if (decode_slice(group_size) == 32) GDN_MT(8, 32, 32);
    GDN_MT(8, 64, 32);
#undef GDN_MT
#undef GDN_ARGS
}

// Workspace bytes launch_decode uses for a call (0: it does not split K).
int64_t decode_workspace_bytes(bool x_f32, int sb_dtype, int M, int N, int K, int bits, int group_size) {
    if (decode_row_blocks(x_f32, M, N, bits, group_size) > 1) return 0;
    const int mt = M <= 16 ? 1 : M <= 32 ? 2 : 4, slice = decode_slice(group_size);
    const int cols = decode_cols(x_f32, mt, bits, group_size);
    const int splits = decode_splits((N + cols - 1) / cols, K / (8 * slice), K, group_size,
                                     sb_dtype == GDN_F32 ? 4 : 8, M, N, INT64_MAX);
    return splits > 1 ? int64_t(splits) * M * N * 4 : 0;
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
                   const void* residual, int M, int N, int K, int group_size, hipStream_t s) {
    const dim3 grid(unsigned((N + BN - 1) / BN), unsigned((M + BM - 1) / BM));
    hipLaunchKernelGGL((qlinear_kernel<BM, BN, kBits, SB, Y>), grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), w,
                       static_cast<const typename SB::storage*>(scales),
                       static_cast<const typename SB::storage*>(biases),
                       static_cast<typename Y::storage*>(y), residual, M, N, K, group_size);
    return check_launch("gdn_quantized_matmul");
}

// Kernel choice for the tiled kernels: 64 x 32 tiles for M <= 64, 128 x 128
// tiles for larger M. (Decode-sized calls the decode kernel takes never get
// here.)
template <int kBits, class SB, class Y>
int dispatch_qlinear(const void* x, const uint32_t* w, const void* scales, const void* biases,
                     void* y, const void* r, int M, int N, int K, int group_size, hipStream_t s) {
    if (M <= 64) return launch_qlinear<64, 32, kBits, SB, Y>(x, w, scales, biases, y, r, M, N, K, group_size, s);
    return launch_qlinear<128, 128, kBits, SB, Y>(x, w, scales, biases, y, r, M, N, K, group_size, s);
}

template <int kBits, class SB>
int dispatch_y(const void* x, const uint32_t* w, const void* scales, const void* biases, void* y,
               int y_dtype, const void* r, int M, int N, int K, int group_size, hipStream_t s) {
    if (y_dtype == GDN_F32) return dispatch_qlinear<kBits, SB, ActF32>(x, w, scales, biases, y, r, M, N, K, group_size, s);
    if (y_dtype == GDN_BF16) return dispatch_qlinear<kBits, SB, ActBF16>(x, w, scales, biases, y, r, M, N, K, group_size, s);
    return dispatch_qlinear<kBits, SB, ActF16>(x, w, scales, biases, y, r, M, N, K, group_size, s);
}

template <int kBits>
int dispatch_sb(const void* x, const uint32_t* w, const void* scales, const void* biases, int sb_dtype,
                void* y, int y_dtype, const void* r, int M, int N, int K, int group_size, hipStream_t s) {
    if (sb_dtype == GDN_F32) return dispatch_y<kBits, ActF32>(x, w, scales, biases, y, y_dtype, r, M, N, K, group_size, s);
    if (sb_dtype == GDN_BF16) return dispatch_y<kBits, ActBF16>(x, w, scales, biases, y, y_dtype, r, M, N, K, group_size, s);
    return dispatch_y<kBits, ActF16>(x, w, scales, biases, y, y_dtype, r, M, N, K, group_size, s);
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

extern "C" int64_t gdn_quantized_matmul_workspace_size(int x_dtype, int sb_dtype, int M, int N, int K, int bits,
                                                       int group_size) {
    const bool x_f32 = x_dtype == GDN_F32;
    if (M < 1 || M > 64 || N < 1 || K < 1 || (bits != 4 && bits != 8) ||
        (group_size != 32 && group_size != 64 && group_size != 128) || K % group_size != 0 ||
        !valid_dtype(sb_dtype) || !(x_dtype == GDN_BF16 || (x_f32 && M <= 32)) ||
        !decode_shape_fits(sb_dtype, N, K, bits, group_size) || gemv_rounds(x_f32, M, K, bits))
        return 0;
    return decode_workspace_bytes(x_f32, sb_dtype, M, N, K, bits, group_size);
}

namespace gdn {
namespace {

int quantized_matmul(const void* x, int x_dtype, const void* w, const void* scales, const void* biases,
                     int sb_dtype, void* y, int y_dtype, const void* residual, int M, int N, int K, int bits,
                     int group_size, void* workspace, int64_t workspace_bytes, void* stream) {
    if (int rc = check_quant_args("gdn_quantized_matmul", w, scales, biases, sb_dtype, N, K, bits,
                                  group_size))
        return rc;
    GDN_REQUIRE(M >= 0, "gdn_quantized_matmul: bad M=%d", M);
    GDN_REQUIRE(valid_dtype(x_dtype) && valid_dtype(y_dtype), "gdn_quantized_matmul: bad dtype");
    GDN_REQUIRE(workspace_bytes >= 0 && reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
                "gdn_quantized_matmul: workspace must be 16-byte aligned");
    const bool x_f32 = x_dtype == GDN_F32;
    if (x_dtype != GDN_BF16 && !(x_f32 && M <= 32))
        return fail(GDN_EUNSUPPORTED,
                    "gdn_quantized_matmul: x must be bfloat16, or float32 with at most 32 rows "
                    "(else use gdn_dequantize)");
    if (M == 0) return 0;
    GDN_REQUIRE(x && y, "gdn_quantized_matmul: null x or y");
    GDN_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0, "gdn_quantized_matmul: x must be 16-byte aligned");
    GDN_REQUIRE(!overlaps(x, int64_t(M) * K * dtype_size(x_dtype), y, int64_t(M) * N * dtype_size(y_dtype)),
                "gdn_quantized_matmul: y overlaps x");
    const int64_t y_bytes = int64_t(M) * N * dtype_size(y_dtype);
    GDN_REQUIRE(!residual || residual == y || !overlaps(residual, y_bytes, y, y_bytes),
                "gdn_quantized_matmul: residual partially overlaps y");
    GDN_REQUIRE(!residual || !overlaps(residual, y_bytes, x, int64_t(M) * K * dtype_size(x_dtype)),
                "gdn_quantized_matmul: residual overlaps x");
    hipStream_t s = as_stream(stream);
    const auto* wp = static_cast<const uint32_t*>(w);
    if (M <= 64 && decode_kernel_fits(x, wp, scales, biases, sb_dtype, N, K, bits, group_size)) {
        if (const int rounds = gemv_rounds(x_f32, M, K, bits))
            return launch_gemv(x, x_f32, wp, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, bits,
                               group_size, rounds, s);
        return launch_decode(x, x_f32, wp, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, bits,
                             group_size, workspace, workspace_bytes, s);
    }
    if (x_f32)
        return fail(GDN_EUNSUPPORTED, "gdn_quantized_matmul: float32 x needs a shape the decode kernel takes");
    if (bits == 4) return dispatch_sb<4>(x, wp, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, group_size, s);
    return dispatch_sb<8>(x, wp, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, group_size, s);
}

// The split-K partial blocks of gdn_quantized_matmul_noalloc live in this
// file-scope device array, one copy per GPU, held until the process ends.
// 4 MiB is the most any call takes: a split call has at most kCUs
// workgroups, so splits * N <= kCUs * 64 columns, and M <= 64 rows of
// float32, i.e. 256 * 64 * 64 * 4 bytes. Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device
// address): it passes the per-device address from hipGetSymbolAddress.
constexpr int64_t kScratchBytes = int64_t(kCUs) * 64 * 64 * 4;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Per device: the scratch's address, and the order of the calls that use
// it. Calls on one stream are ordered by the stream; a call on another
// stream than the previous scratch user's first waits (on the GPU) for the
// event recorded after that call, so calls from several streams take the
// scratch in turn instead of racing on it. Calls made while their stream
// is being captured into a graph neither wait nor record (a capture may
// not wait on work outside it): a graph's replays are ordered against
// eager calls on other streams by the caller.
struct ScratchState {
    void* ptr = nullptr;
    hipEvent_t done = nullptr;          // recorded after the last eager scratch user
    hipStream_t last = nullptr;         // that call's stream
    bool used = false;
};
std::mutex g_scratch_mutex;
ScratchState g_scratch[kMaxDevices];

// Set-up on the first call on a device, with that device current: the
// scratch array's address (hipGetSymbolAddress) and the ordering event.
int scratch_setup(int dev, ScratchState& st) {
    int current = -1;
    hipError_t err = hipGetDevice(&current);
    if (err == hipSuccess && current != dev) err = hipSetDevice(dev);
    void* p = nullptr;
    if (err == hipSuccess) err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    hipEvent_t ev = nullptr;
    if (err == hipSuccess) err = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (current >= 0 && current != dev) {
        const hipError_t back = hipSetDevice(current);
        if (err == hipSuccess) err = back;
    }
    if (err != hipSuccess || !p)
        return fail(err != hipSuccess ? int(err) : GDN_EINVAL,
                    "gdn_quantized_matmul_noalloc: scratch set-up on device %d: %s", dev, hipGetErrorString(err));
    st.ptr = p;
    st.done = ev;
    return 0;
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_quantized_matmul(const void* x, int x_dtype, const void* w, const void* scales,
                                    const void* biases, int sb_dtype, void* y, int y_dtype,
                                    const void* residual, int M, int N, int K, int bits, int group_size,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
    return quantized_matmul(x, x_dtype, w, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, bits,
                            group_size, workspace, workspace_bytes, stream);
}

extern "C" int gdn_quantized_matmul_noalloc(const void* x, int x_dtype, const void* w, const void* scales,
                                            const void* biases, int sb_dtype, void* y, int y_dtype,
                                            const void* residual, int M, int N, int K, int bits,
                                            int group_size, void* stream) {
    const int64_t need = gdn_quantized_matmul_workspace_size(x_dtype, sb_dtype, M, N, K, bits, group_size);
    if (need > kScratchBytes)
        return fail(GDN_EINVAL,
                    "gdn_quantized_matmul_noalloc: this call needs %lld bytes of split-K scratch; the "
                    "library holds %lld (use gdn_quantized_matmul with a workspace)",
                    static_cast<long long>(need), static_cast<long long>(kScratchBytes));
    if (need == 0)  // no split: the scratch is not touched
        return quantized_matmul(x, x_dtype, w, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, bits,
                                group_size, nullptr, 0, stream);
    const hipStream_t s = as_stream(stream);
    int dev = -1;
    hipError_t err = hipStreamGetDevice(s, &dev);
    if (err != hipSuccess)
        return fail(int(err), "gdn_quantized_matmul_noalloc: hipStreamGetDevice: %s", hipGetErrorString(err));
    GDN_REQUIRE(dev >= 0 && dev < kMaxDevices, "gdn_quantized_matmul_noalloc: device %d out of range", dev);
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    err = hipStreamIsCapturing(s, &capture);
    if (err != hipSuccess)
        return fail(int(err), "gdn_quantized_matmul_noalloc: hipStreamIsCapturing: %s", hipGetErrorString(err));
    const bool eager = capture == hipStreamCaptureStatusNone;
    // held from the wait to the record, so that calls from several host
    // threads take the scratch in the order they enqueue
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ScratchState& st = g_scratch[dev];
    if (!st.ptr)
        if (int rc = scratch_setup(dev, st)) return rc;
    if (eager && st.used && st.last != s) {
        err = hipStreamWaitEvent(s, st.done, 0);
        if (err != hipSuccess)
            return fail(int(err), "gdn_quantized_matmul_noalloc: hipStreamWaitEvent: %s", hipGetErrorString(err));
    }
    const int rc = quantized_matmul(x, x_dtype, w, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K,
                                    bits, group_size, st.ptr, need, stream);
    if (rc != 0 || !eager) return rc;
    err = hipEventRecord(st.done, s);
    if (err != hipSuccess)
        return fail(int(err), "gdn_quantized_matmul_noalloc: hipEventRecord: %s", hipGetErrorString(err));
    st.last = s;
    st.used = true;
    return 0;
}

namespace gdn {
namespace {

// The microscaling float codes (OCP MX formats): e2m1 (fp4: sign, 2-bit
// exponent of bias 1, 1-bit mantissa; exponent 0 is 0 or 0.5), e4m3 (fp8:
// sign, 4-bit exponent of bias 7, 3-bit mantissa; exponent 0 subnormal,
// 0x7F / 0xFF NaN) and e8m0 (a power of two, 2^(c - 127); 255 NaN).
GDN_DEV float e2m1_value(uint32_t c) {
    const int e = int(c >> 1) & 3;
    const float mag = e == 0 ? 0.5f * float(c & 1) : ldexpf(1.f + 0.5f * float(c & 1), e - 1);
    return (c & 8) ? -mag : mag;
}

GDN_DEV float e4m3_value(uint32_t c) {
    const int e = int(c >> 3) & 15, m = int(c & 7);
    if (e == 15 && m == 7) return __builtin_nanf("");
    const float mag = e == 0 ? ldexpf(float(m), -9) : ldexpf(1.f + float(m) * 0.125f, e - 7);
    return (c & 0x80) ? -mag : mag;
}

GDN_DEV float e8m0_value(uint32_t c) { return c == 255 ? __builtin_nanf("") : ldexpf(1.f, int(c) - 127); }

// Dense weights of any scheme QuantScheme accepts, one thread per 32
// elements of a row (the last may hold 16): element k of a row is the
// bits-wide field at bit bits * k of the row's little-endian bit stream
// (MLX packs 3-, 5- and 6-bit codes into byte groups, which reads the same),
// so a thread's 32 codes are its `bits` consecutive words. affine:
// s * q + b in float32, rounded once to out's dtype; mxfp4 / mxfp8 / nvfp4:
// the code's value times the group's scale (e8m0, or e4m3 for nvfp4), exact
// in float32 and in bf16 (at most 6 significant bits).
__global__ __launch_bounds__(256) void dequantize_scheme_kernel(
    const uint32_t* __restrict__ w, const void* __restrict__ scales, const void* __restrict__ biases,
    int sb_dtype, void* __restrict__ out, int out_dtype, int N, int K, int bits, int group_size, int mode) {
    const int chunks = (K + 31) / 32;
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= int64_t(N) * chunks) return;
    const int n = int(t / chunks), k0 = int(t % chunks) * 32;
    const int64_t row_words = int64_t(K) * bits / 32;
    const uint32_t* rw = w + int64_t(n) * row_words + int64_t(k0) * bits / 32;
    const int words = int((int64_t(K - k0 < 32 ? K - k0 : 32) * bits + 31) / 32);
    uint32_t wd[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) wd[i] = i < words ? rw[i] : 0u;
    const uint32_t mask = (1u << bits) - 1u;
    const int gpr = K / group_size;
    const int64_t sb_row = int64_t(n) * gpr;
    for (int e = 0; e < 32 && k0 + e < K; ++e) {
        const int off = bits * e, wi = off >> 5, sh = off & 31;
        const uint64_t pair = uint64_t(wd[wi]) | (uint64_t(wd[wi + 1]) << 32);
        const uint32_t q = uint32_t(pair >> sh) & mask;
        const int64_t g = sb_row + (k0 + e) / group_size;
        float v;
        if (mode == GDN_QUANT_AFFINE) {
            v = __builtin_fmaf(load_any(scales, g, sb_dtype), float(q), load_any(biases, g, sb_dtype));
        } else {
            const uint32_t sc = static_cast<const uint8_t*>(scales)[g];
            const float code = mode == GDN_QUANT_MXFP8 ? e4m3_value(q) : e2m1_value(q);
            v = code * (mode == GDN_QUANT_NVFP4 ? e4m3_value(sc) : e8m0_value(sc));
        }
        store_any(out, int64_t(n) * K + k0 + e, out_dtype, v);
    }
}

// ---- every scheme at decode sizes ---------------------------------------
//
// A lane's codes for one "super block" of 32 kU k (kU MFMA k blocks): lane
// l takes the 8 kU consecutive codes from k_sb + 8 kU (l / 16) of column
// l % 16 and gives codes 8u .. 8u + 7 to MFMA u; x's A operand takes the
// same k order (its 8 kU values from the same k, 16 kU contiguous bytes per
// row), so each MFMA still sums x times W over 32 k. The lane's codes are
// one run of kLen = 8 kU kBits bits from bit kBits k_lane of the row. Runs
// of a super block start kLen bits apart, so a run starts kLen g % 32 bits
// into a word (lane group g); kNW words hold the run at the largest such
// offset. Runs starting on a word (kAligned) are whole words; the others are
// shifted into place first (a funnel shift per word). All but the last of
// the kNW words hold bits of the run; the last may lie past the row for the
// row's final run, and its index is clamped.
template <int kBits, int kU>
struct SchemeRun {
    static constexpr int kLen = 8 * kU * kBits;
    static constexpr int kShMax = (kLen % 32) > (2 * kLen % 32)
                                      ? ((kLen % 32) > (3 * kLen % 32) ? kLen % 32 : 3 * kLen % 32)
                                      : ((2 * kLen % 32) > (3 * kLen % 32) ? 2 * kLen % 32 : 3 * kLen % 32);
    static constexpr bool kAligned = kShMax == 0;
    static constexpr int kNW = (kShMax + kLen + 31) / 32;
};

// Code c of a lane's run (c a compile-time constant after unrolling).
template <int kBits>
GDN_DEV uint32_t run_code(const uint32_t* wd, int c) {
    const int p = kBits * c, w = p >> 5, s = p & 31;
    const uint32_t v = s + kBits <= 32 ? wd[w] >> s : __builtin_amdgcn_alignbit(wd[w + 1], wd[w], s);
    return v & ((1u << kBits) - 1u);
}

// Codes 8u .. 8u + 7 of a lane's run as the MFMA's bf16 B operand:
//   affine, 2-6 bits: the bf16 bits 0x4300 | q, i.e. 128 + q (exact; the
//     host's bias is b - 128 s); 8 bits: q;
//   mxfp4 / mxfp8: the e2m1 / e4m3 values times the group's scale 2^(e - 127)
//     (gfx950's scaled conversions, which take the scale's exponent: exact);
//   nvfp4: e2m1 values times the e4m3 scale of each code's 16-code group
//     (sc0 for codes 0-15 of the run, sc1 for 16-31), exact in bf16.
template <int kMode, int kBits>
GDN_DEV bf16x8 run_fragment(const uint32_t* wd, int u, float sc0, float sc1) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 d;
    if constexpr (kMode == GDN_QUANT_AFFINE && kBits <= 6) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            d[i] = (run_code<kBits>(wd, 8 * u + 2 * i) | run_code<kBits>(wd, 8 * u + 2 * i + 1) << 16) | 0x43004300u;
    } else if constexpr (kMode == GDN_QUANT_AFFINE) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            d[i] = pack_bf16x2(float(run_code<kBits>(wd, 8 * u + 2 * i)), float(run_code<kBits>(wd, 8 * u + 2 * i + 1)));
    } else if constexpr (kMode == GDN_QUANT_MXFP4) {
        // byte i of the word: its low nibble to the low half
        const uint32_t q = wd[u];
        d[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc0, 0));
        d[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc0, 1));
        d[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc0, 2));
        d[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc0, 3));
    } else if constexpr (kMode == GDN_QUANT_MXFP8) {
        // 16-bit half of a word: its low byte to the low half
        const uint32_t q0 = wd[2 * u], q1 = wd[2 * u + 1];
        d[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q0, sc0, false));
        d[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q0, sc0, true));
        d[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q1, sc0, false));
        d[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q1, sc0, true));
    } else {
        const float sc = u < 2 ? sc0 : sc1;
        const uint32_t q = wd[u];
        const auto f0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q, 1.0f, 0);
        const auto f1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q, 1.0f, 1);
        const auto f2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q, 1.0f, 2);
        const auto f3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q, 1.0f, 3);
        d[0] = pack_bf16x2(f0[0] * sc, f0[1] * sc);
        d[1] = pack_bf16x2(f1[0] * sc, f1[1] * sc);
        d[2] = pack_bf16x2(f2[0] * sc, f2[1] * sc);
        d[3] = pack_bf16x2(f3[0] * sc, f3[1] * sc);
    }
    return __builtin_bit_cast(bf16x8, d);
}

constexpr int kSchemeWaves = 8;   // waves of a workgroup, dealt the super blocks in turn
constexpr int kSchemeMaxSplits = 16;
// groups of a column one split may span: (s, b) float pairs for affine
// codes, one float for the others; rows of the LDS table are one entry
// longer (fewer bank conflicts)
constexpr int kSchemeGroupsAffine = 128;
constexpr int kSchemeGroupsFloat = 256;
static_assert((kSchemeGroupsFloat + 1) * 4 <= (kSchemeGroupsAffine + 1) * 8, "LDS share of the scales");

// Output columns of a workgroup: 64 (four MFMA column tiles), or 32 where
// 64-column tiles would number fewer than 128 (K is then split more finely
// instead: measured on 2048 x 4096 weights, 32 columns in 4 splits take
// 7.5-8.8 us at one row and 14-16 us at 64 rows against 8-13 and 19-22 us
// for 64 columns in 8; on 12352 x 2048, 64 columns take 22 us at 64 rows
// against 31 us for 32).
int scheme_cols(int N) { return (N + 63) / 64 < 128 ? 32 : 64; }

// y = x W^T for M <= 64 bf16 rows and the packed codes of any scheme
// (mx.quantized_matmul at decode sizes, model/moe_block.py:44-55), reading
// the weight once at its packed size. A workgroup of 8 waves takes kCols
// columns (16-column MFMA tiles) and the k range of split blockIdx.y
// (all of K with one split). Its columns' scales (and biases) for the range
// are first converted to float in LDS; the range's super blocks are then
// dealt to the waves in turn, each lane loading its run of codes per column
// tile and its x values per row tile (rows clamped to M - 1, never stored)
// straight into registers, two super blocks in flight. Per super block and
// output (m, n), with the run's bf16 values v (run_fragment):
//   affine:       y += s P + b' X, P = sum x v, X = sum x (a product against
//                 ones), b' = b - 128 s for 2-6-bit codes: float32 sums
//                 with scale and bias per super block (within one group),
//                 as MLX's matrix-vector kernels apply them per group;
//   mxfp4, mxfp8, nvfp4: y += sum x v, the scale being in v.
// The 8 waves' float32 blocks are added in LDS in wave order. With S > 1
// splits the sum goes to partial[split][M][N] (qlinear_split_sum_kernel adds
// the splits in order), else to y with the residual. The host guarantees:
// K / 32 / S a multiple of kU, 32 kU <= group_size for affine codes, the
// split's groups within the LDS share, 16-byte aligned x.
template <int kMode, int kBits, int kMT, int kU, int kCols>
__global__ __launch_bounds__(512) void qlinear_scheme_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w, const void* __restrict__ scales,
    const void* __restrict__ biases, int sb_dtype, void* y, int y_dtype, const void* residual,
    float* __restrict__ partial, int M, int N, int K, int group_size) {
    using Run = SchemeRun<kBits, kU>;
    constexpr bool kAffine = kMode == GDN_QUANT_AFFINE;
    constexpr int kCT = kCols / 16;
    constexpr int kSlots = kMT * kCT;  // float4 accumulators per lane
    constexpr int kRedBytes = kSchemeWaves * kSlots * 64 * 16;
    constexpr int kSBBytes = kCols * (kSchemeGroupsAffine + 1) * 8;
    constexpr int kLds = kRedBytes > kSBBytes ? kRedBytes : kSBBytes;
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
    float* sbl = reinterpret_cast<float*>(lds);  // [kCols][G + 1] floats or float pairs

    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, g = l >> 4, n = l & 15;
    const int n0 = blockIdx.x * kCols;
    const int64_t row_words = int64_t(K) * kBits / 32;
    const int gpr = K / group_size;
    const int kspan = K / gridDim.y, kbase = blockIdx.y * kspan;  // this split's k range
    const int G = kspan / group_size, gstride = G + 1;            // its groups per column

    // the split's scales (and biases) of the workgroup's columns, as float:
    // 512 / kCols threads per column take its groups in turn, requesting 8
    // entries at a time (one memory latency per 8, not per entry); the
    // scales' dtype is resolved outside the loop
    auto stage_scales = [&]() {
        constexpr int kTPC = 512 / kCols, kB = 8;
        const int c = tid / kTPC, j0 = tid % kTPC;
        const int col = n0 + c < N ? n0 + c : N - 1;
        const int64_t src0 = int64_t(col) * gpr + kbase / group_size;
        float* row = sbl + (kAffine ? 2 : 1) * c * gstride;
        auto stage = [&](auto to_float) {
            for (int g0 = j0; g0 < G; g0 += kTPC * kB) {
                decltype(to_float(0)) sv[kB], bv[kB];
#pragma unroll
                for (int j = 0; j < kB; ++j) {
                    const int gi = g0 + kTPC * j;
                    if (gi < G) {
                        sv[j] = to_float(src0 + gi);
                        if constexpr (kAffine) bv[j] = to_float(~(src0 + gi));
                    }
                }
#pragma unroll
                for (int j = 0; j < kB; ++j) {
                    const int gi = g0 + kTPC * j;
                    if (gi < G) {
                        if constexpr (kAffine) {
                            const float sf = float(sv[j]), bf = float(bv[j]);
                            const float b2 = kBits <= 6 ? __builtin_fmaf(-128.f, sf, bf) : bf;
                            *reinterpret_cast<float2*>(row + 2 * gi) = float2{sf, b2};
                        } else {
                            row[gi] = float(sv[j]);
                        }
                    }
                }
            }
        };
        // entry i of the scales, or of the biases when passed ~i
        if constexpr (kAffine) {
            const auto* s32 = static_cast<const float*>(scales);
            const auto* b32 = static_cast<const float*>(biases);
            const auto* s16 = static_cast<const uint16_t*>(scales);
            const auto* b16 = static_cast<const uint16_t*>(biases);
            if (sb_dtype == GDN_F32)
                stage([&](int64_t i) { return i >= 0 ? s32[i] : b32[~i]; });
            else if (sb_dtype == GDN_BF16)
                stage([&](int64_t i) { return bf16_bits_to_f32(i >= 0 ? s16[i] : b16[~i]); });
            else
                stage([&](int64_t i) { return f16_bits_to_f32(i >= 0 ? s16[i] : b16[~i]); });
        } else {
            // mx: the float whose exponent field is the e8m0 code (the
            // conversions read only the exponent)
            const auto* s8 = static_cast<const uint8_t*>(scales);
            stage([&](int64_t i) {
                const uint32_t code = s8[i];
                return kMode == GDN_QUANT_NVFP4 ? e4m3_value(code) : __uint_as_float(code << 23);
            });
        }
    };

    const uint32_t* wrow[kCT];
#pragma unroll
    for (int ct = 0; ct < kCT; ++ct) {
        const int c = n0 + 16 * ct + n < N ? n0 + 16 * ct + n : N - 1;
        wrow[ct] = w + c * row_words;
    }
    const uint16_t* xrow[kMT];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) xrow[mt] = x + int64_t(16 * mt + n < M ? 16 * mt + n : M - 1) * K;

    // this split's super blocks; the wave's are wv + 8 i, i < nbw
    const int nsb = kspan / (32 * kU);
    const int nbw = nsb > wv ? (nsb - wv + kSchemeWaves - 1) / kSchemeWaves : 0;
    const int last = nbw > 0 ? wv + kSchemeWaves * (nbw - 1) : 0;

    struct Slot {
        uint32_t wd[kCT][Run::kNW];
        u16x8 xv[kMT][kU];
        int k;  // the lane's first k (from the split's start)
    };
    auto load = [&](Slot& sl, int i) {
        const int sb = wv + kSchemeWaves * i < last ? wv + kSchemeWaves * i : last;
        const int kl = 32 * kU * sb + 8 * kU * g;
        sl.k = kl;
        const int64_t off = int64_t(kBits) * (kbase + kl), wi = off >> 5;
        const int64_t wl = wi + Run::kNW - 1, wlc = Run::kAligned || wl < row_words ? wl : row_words - 1;
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) {
#pragma unroll
            for (int j = 0; j + 1 < Run::kNW; ++j) sl.wd[ct][j] = wrow[ct][wi + j];
            sl.wd[ct][Run::kNW - 1] = wrow[ct][wlc];
        }
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
            for (int u = 0; u < kU; ++u) sl.xv[mt][u] = *reinterpret_cast<const u16x8*>(xrow[mt] + kbase + kl + 8 * u);
    };

    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc[kMT][kCT];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) acc[mt][ct] = zero;
    bf16x8 ones;
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = static_cast<__bf16>(1.0f);

    auto compute = [&](Slot& sl) {
        const int sh = int((int64_t(kBits) * (kbase + sl.k)) & 31);
        const int gl = sl.k / group_size;  // the run's (first) group in the split
        f32x4 X[kMT];
        if constexpr (kAffine) {
#pragma unroll
            for (int mt = 0; mt < kMT; ++mt) {
                X[mt] = zero;
#pragma unroll
                for (int u = 0; u < kU; ++u) X[mt] = mfma_bf16(__builtin_bit_cast(bf16x8, sl.xv[mt][u]), ones, X[mt]);
            }
        }
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) {
            uint32_t* wd = sl.wd[ct];
            if constexpr (!Run::kAligned) {
#pragma unroll
                for (int j = 0; j + 1 < Run::kNW; ++j) wd[j] = __builtin_amdgcn_alignbit(wd[j + 1], wd[j], sh);
                wd[Run::kNW - 1] >>= sh;  // the run's bits in the last word
            }
            const float* se = sbl + (kAffine ? 2 : 1) * ((16 * ct + n) * gstride + gl);
            float sc0 = 0.f, sc1 = 0.f, s = 0.f, b = 0.f;
            if constexpr (kAffine) {
                const float2 sbv = *reinterpret_cast<const float2*>(se);
                s = sbv.x;
                b = sbv.y;
            } else {
                sc0 = se[0];
                if constexpr (kMode == GDN_QUANT_NVFP4) sc1 = kU == 4 ? se[1] : sc0;
            }
            bf16x8 bq[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) bq[u] = run_fragment<kMode, kBits>(wd, u, sc0, sc1);
#pragma unroll
            for (int mt = 0; mt < kMT; ++mt) {
                if constexpr (kAffine) {
                    f32x4 P = zero;
#pragma unroll
                    for (int u = 0; u < kU; ++u) P = mfma_bf16(__builtin_bit_cast(bf16x8, sl.xv[mt][u]), bq[u], P);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[mt][ct][i] = __builtin_fmaf(b, X[mt][i], __builtin_fmaf(s, P[i], acc[mt][ct][i]));
                } else {
#pragma unroll
                    for (int u = 0; u < kU; ++u)
                        acc[mt][ct] = mfma_bf16(__builtin_bit_cast(bf16x8, sl.xv[mt][u]), bq[u], acc[mt][ct]);
                }
            }
        }
    };

    // Two super blocks in flight: block i in slot i % 2. The first two
    // blocks' operands are requested before the scales, so that one memory
    // latency covers both. Requests carry no condition (a slot's registers
    // are then free between its compute and its next load) and never
    // re-request a block read earlier (that can miss L2 again): past the
    // wave's last block, load's clamp gives the last block, which the other
    // slot requested just before, so the two misses meet in L2.
    Slot ring[2];
    load(ring[0], 0);
    load(ring[1], 1);
    stage_scales();
    __syncthreads();  // the scales are in LDS
    int i0 = 0;
    for (; i0 + 2 < nbw; i0 += 2) {
        // the fences keep each load after the compute that frees its slot
        compute(ring[0]);
        __builtin_amdgcn_sched_barrier(0);
        load(ring[0], i0 + 2);
        compute(ring[1]);
        __builtin_amdgcn_sched_barrier(0);
        load(ring[1], i0 + 3);
    }
    if (i0 < nbw) compute(ring[0]);
    if (i0 + 1 < nbw) compute(ring[1]);

    // the waves' blocks added in wave order; thread t then owns accumulator
    // slots t, t + 512, ... (slot = (mt kCT + ct) 64 + lane)
    __syncthreads();  // every wave is done with the scales
    f32x4* red = reinterpret_cast<f32x4*>(lds);
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) red[(wv * kSlots + mt * kCT + ct) * 64 + l] = acc[mt][ct];
    __syncthreads();
    for (int q = tid; q < kSlots * 64; q += 512) {
        f32x4 v = red[q];
#pragma unroll
        for (int ww = 1; ww < kSchemeWaves; ++ww) v += red[ww * kSlots * 64 + q];
        const int slot = q >> 6, lane = q & 63, mt = slot / kCT, ct = slot % kCT;
        const int col = n0 + 16 * ct + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * mt + 4 * (lane >> 4) + i;
            if (row < M && col < N) {
                const int64_t o = int64_t(row) * N + col;
                if (partial) partial[int64_t(blockIdx.y) * M * N + o] = v[i];
                else store_any(y, o, y_dtype, plus_residual(v[i], residual, o, y_dtype));
            }
        }
    }
}

// Splits of K for `tiles` column tiles and nb 32-k blocks: the largest
// power of two S <= 16 leaving each split a multiple of 4 blocks and at
// least kSchemeMinBlocks of them, at most 256 workgroups (one per CU) and
// S M N floats of workspace.
constexpr int kSchemeMinBlocks = 16;
int scheme_splits(int tiles, int nb, int M, int N, int64_t ws_bytes) {
    int best = 1;
    for (int sp = 2; sp <= kSchemeMaxSplits; sp *= 2) {
        if (nb % (4 * sp) != 0 || nb / sp < kSchemeMinBlocks || int64_t(tiles) * sp > kCUs ||
            int64_t(sp) * M * N * 4 > ws_bytes)
            break;
        best = sp;
    }
    return best;
}

template <int kMode, int kBits>
int launch_scheme(const void* x, const uint32_t* w, const void* scales, const void* biases, int sb_dtype,
                  void* y, int y_dtype, const void* residual, int M, int N, int K, int group_size,
                  void* workspace, int64_t ws_bytes, hipStream_t s) {
    const int cols = scheme_cols(N), tiles = (N + cols - 1) / cols, nb = K / 32;
    const int splits = scheme_splits(tiles, nb, M, N, workspace ? ws_bytes : 0);
    const int groups = K / splits / group_size;
    GDN_REQUIRE(groups <= (kMode == GDN_QUANT_AFFINE ? kSchemeGroupsAffine : kSchemeGroupsFloat),
                "gdn_quantized_matmul_scheme: %d groups of a column in one split (K too long for the "
                "workspace given)", groups);
    float* partial = splits > 1 ? static_cast<float*>(workspace) : nullptr;
    if (partial)
        GDN_REQUIRE(!overlaps(partial, int64_t(splits) * M * N * 4, y, int64_t(M) * N * dtype_size(y_dtype)) &&
                        !overlaps(partial, int64_t(splits) * M * N * 4, x, int64_t(M) * K * 2) &&
                        (!residual || !overlaps(partial, int64_t(splits) * M * N * 4, residual,
                                                int64_t(M) * N * dtype_size(y_dtype))),
                    "gdn_quantized_matmul_scheme: workspace overlaps x, y or residual");
    // super blocks of kU MFMA blocks: up to 4 (2 with 64 rows: registers),
    // within one group for affine codes, dividing the split's blocks
    const int per_split = nb / splits;
    int ku = M > 16 ? 2 : 4;
    if (kMode == GDN_QUANT_AFFINE) ku = ku < group_size / 32 ? ku : group_size / 32;
    while (per_split % ku != 0) ku /= 2;
    const dim3 grid{unsigned(tiles), unsigned(splits)};
    const auto* xp = static_cast<const uint16_t*>(x);
#define GDN_SCHEME_C(MT, U, C)                                                                              \
    hipLaunchKernelGGL((qlinear_scheme_kernel<kMode, kBits, MT, U, C>), grid, dim3(512), 0, s, xp, w, scales, \
                       biases, sb_dtype, y, y_dtype, residual, partial, M, N, K, group_size)
#define GDN_SCHEME(MT, U)              \
    do {                               \
        if (cols == 32)                \
            GDN_SCHEME_C(MT, U, 32);   \
        else                           \
            GDN_SCHEME_C(MT, U, 64);   \
    } while (0)
    if (M <= 16) {
        if (ku == 4) GDN_SCHEME(1, 4);
        else if (ku == 2) GDN_SCHEME(1, 2);
        else GDN_SCHEME(1, 1);
    } else if constexpr (kMode == GDN_QUANT_AFFINE && kBits == 8) {
        GDN_SCHEME(4, 1);  // two 8-bit super blocks in flight would spill
    } else {
        if (ku == 2) GDN_SCHEME(4, 2);
        else GDN_SCHEME(4, 1);
    }
#undef GDN_SCHEME
#undef GDN_SCHEME_C
    if (int rc = check_launch("gdn_quantized_matmul_scheme")) return rc;
    if (!partial) return 0;
    return launch_split_sum(partial, splits, int64_t(M) * N, y, y_dtype, residual, s, "gdn_quantized_matmul_scheme");
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_dequantize(const void* w, const void* scales, const void* biases, int sb_dtype,
                              void* out, int out_dtype, int N, int K, int bits, int group_size, int mode,
                              void* stream) {
    GDN_REQUIRE(out && valid_dtype(out_dtype), "gdn_dequantize: bad output");
    hipStream_t s = as_stream(stream);
    if (mode == GDN_QUANT_AFFINE && (bits == 4 || bits == 8)) {
        if (int rc = check_quant_args("gdn_dequantize", w, scales, biases, sb_dtype, N, K, bits, group_size))
            return rc;
        const auto* wp = static_cast<const uint32_t*>(w);
        if (bits == 4) return launch_dequant<4>(wp, scales, biases, sb_dtype, out, out_dtype, N, K, group_size, s);
        return launch_dequant<8>(wp, scales, biases, sb_dtype, out, out_dtype, N, K, group_size, s);
    }
    // the schemes of the reference's QuantScheme (config.py:17-33)
    bool ok;
    switch (mode) {
        case GDN_QUANT_AFFINE:
            ok = (bits >= 2 && bits <= 8 && bits != 7) &&
                 (group_size == 32 || group_size == 64 || group_size == 128);
            break;
        case GDN_QUANT_MXFP4: ok = bits == 4 && group_size == 32; break;
        case GDN_QUANT_MXFP8: ok = bits == 8 && group_size == 32; break;
        case GDN_QUANT_NVFP4: ok = bits == 4 && group_size == 16; break;
        default: ok = false;
    }
    GDN_REQUIRE(ok, "gdn_dequantize: mode %d with bits=%d, group_size=%d is not a scheme", mode, bits,
                group_size);
    GDN_REQUIRE(N > 0 && K > 0 && K % group_size == 0 && int64_t(K) * bits % 32 == 0,
                "gdn_dequantize: K=%d must be a multiple of group_size and fill whole words", K);
    GDN_REQUIRE(w && scales && (mode != GDN_QUANT_AFFINE || biases), "gdn_dequantize: null weight, scales or biases");
    GDN_REQUIRE(mode != GDN_QUANT_AFFINE || valid_dtype(sb_dtype), "gdn_dequantize: bad scales/biases dtype");
    const int64_t threads = int64_t(N) * ((K + 31) / 32);
    GDN_REQUIRE(threads < (int64_t(1) << 31), "gdn_dequantize: %lld elements exceed the grid",
                (long long)N * K);
    hipLaunchKernelGGL(dequantize_scheme_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s,
                       static_cast<const uint32_t*>(w), scales, biases, sb_dtype, out, out_dtype, N, K, bits,
                       group_size, mode);
    return check_launch("gdn_dequantize");
}

extern "C" int64_t gdn_quantized_matmul_scheme_workspace_size(int M, int N, int K) {
    if (M <= 0 || M > 64 || N <= 0 || K <= 0 || K % 32 != 0) return 0;
    const int cols = scheme_cols(N);
    const int splits = scheme_splits((N + cols - 1) / cols, K / 32, M, N, INT64_MAX);
    return splits > 1 ? int64_t(splits) * M * N * 4 : 0;
}

extern "C" int gdn_quantized_matmul_scheme(const void* x, const void* w, const void* scales, const void* biases,
                                           int sb_dtype, void* y, int y_dtype, const void* residual, int M, int N,
                                           int K, int bits, int group_size, int mode, void* workspace,
                                           int64_t workspace_bytes, void* stream) {
    bool ok;
    switch (mode) {  // the schemes of the reference's QuantScheme (config.py:17-33)
        case GDN_QUANT_AFFINE:
            ok = (bits >= 2 && bits <= 8 && bits != 7) && (group_size == 32 || group_size == 64 || group_size == 128);
            break;
        case GDN_QUANT_MXFP4: ok = bits == 4 && group_size == 32; break;
        case GDN_QUANT_MXFP8: ok = bits == 8 && group_size == 32; break;
        case GDN_QUANT_NVFP4: ok = bits == 4 && group_size == 16; break;
        default: ok = false;
    }
    GDN_REQUIRE(ok, "gdn_quantized_matmul_scheme: mode %d with bits=%d, group_size=%d is not a scheme", mode,
                bits, group_size);
    GDN_REQUIRE(M >= 0 && M <= 64, "gdn_quantized_matmul_scheme: M=%d (1 to 64 rows)", M);
    GDN_REQUIRE(N > 0 && K > 0 && K % 32 == 0 && K % group_size == 0,
                "gdn_quantized_matmul_scheme: K=%d must be a multiple of 32 and of group_size", K);
    GDN_REQUIRE(int64_t(N) * K * bits / 8 < (int64_t(1) << 31), "gdn_quantized_matmul_scheme: weight too large");
    GDN_REQUIRE(valid_dtype(y_dtype), "gdn_quantized_matmul_scheme: bad y dtype");
    GDN_REQUIRE(mode != GDN_QUANT_AFFINE || valid_dtype(sb_dtype), "gdn_quantized_matmul_scheme: bad scales dtype");
    if (M == 0) return 0;
    GDN_REQUIRE(x && w && scales && y && (mode != GDN_QUANT_AFFINE || biases),
                "gdn_quantized_matmul_scheme: null pointer");
    GDN_REQUIRE((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16 == 0,
                "gdn_quantized_matmul_scheme: x and w must be 16-byte aligned");
    const int64_t y_bytes = int64_t(M) * N * dtype_size(y_dtype);
    GDN_REQUIRE(!overlaps(x, int64_t(M) * K * 2, y, y_bytes), "gdn_quantized_matmul_scheme: y overlaps x");
    GDN_REQUIRE(!residual || residual == y || !overlaps(residual, y_bytes, y, y_bytes),
                "gdn_quantized_matmul_scheme: residual partially overlaps y");
    hipStream_t s = as_stream(stream);
    const auto* wp = static_cast<const uint32_t*>(w);
    GDN_REQUIRE(!workspace || reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
                "gdn_quantized_matmul_scheme: workspace must be 16-byte aligned");
#define GDN_ARGS x, wp, scales, biases, sb_dtype, y, y_dtype, residual, M, N, K, group_size, workspace, workspace_bytes, s
    switch (mode) {
        case GDN_QUANT_MXFP4: return launch_scheme<GDN_QUANT_MXFP4, 4>(GDN_ARGS);
        case GDN_QUANT_MXFP8: return launch_scheme<GDN_QUANT_MXFP8, 8>(GDN_ARGS);
        case GDN_QUANT_NVFP4: return launch_scheme<GDN_QUANT_NVFP4, 4>(GDN_ARGS);
        default: break;
    }
    switch (bits) {
        case 2: return launch_scheme<GDN_QUANT_AFFINE, 2>(GDN_ARGS);
        case 3: return launch_scheme<GDN_QUANT_AFFINE, 3>(GDN_ARGS);
        case 4: return launch_scheme<GDN_QUANT_AFFINE, 4>(GDN_ARGS);
        case 5: return launch_scheme<GDN_QUANT_AFFINE, 5>(GDN_ARGS);
        case 6: return launch_scheme<GDN_QUANT_AFFINE, 6>(GDN_ARGS);
        default: return launch_scheme<GDN_QUANT_AFFINE, 8>(GDN_ARGS);
    }
#undef GDN_ARGS
}
