// Chunked (WY / UT) prefill of the gated-delta recurrence on bf16 MFMA.
//
// The reference prefills with the sequential recurrence
// (_gated_delta_metal.py:64-87, gated_delta.py:93-109). Over a chunk of C = 64
// tokens with start state S0 (Dv x Dk), log-decay l_i = sum_{j<=i} log g_j and
// G_ij = exp(l_i - l_j), the same recurrence is
//
//   A   = strict_lower(diag(beta) (K K^T) o G),   Tb = (I + A)^-1 diag(beta)
//   R   = V - diag(exp l) K S0^T,                 D  = Tb R        (per-token deltas)
//   Y   = diag(exp l) Q S0^T + lower(Q K^T o G) D
//   S_C = exp(l_C) S0 + (diag(exp(l_C - l)) D)^T K
//
// Two kernels:
//   chunk pass (parallel over chunks x key heads): K K^T and Q K^T on MFMA,
//     the gates, the blocked triangular inverse, and per value head the
//     records Tb and P = lower(Q K^T o G) (each bf16 hi + lo) plus exp(l)
//     and exp(l_C - l).
//   state pass (per run x value head x 16-row slice of the state, sequential
//     over the run's chunks): K S^T and Q S^T, Tb R, P D and the state update
//     on MFMA, the state tile resident in accumulators.
//
// Operands that are exact in bf16 (q, k, v) enter the MFMAs as they are;
// float32 operands (S, Tb, R, P, D) are split into a bf16 high part and a
// bf16 residual, with the residual products added (hi.hi + hi.lo + lo.hi),
// which keeps state and output within ~1e-5 relative of the sequential
// recurrence.
//
// MFMA: v_mfma_f32_16x16x32_bf16. Lane l holds A[l%16][8(l/16)+j],
// B[8(l/16)+j][l%16] (j = 0..7) and D[4(l/16)+i][l%16] (i = 0..3).
#include "gdn_common.h"
#include "gdn_conv.h"
#include "gdn_host.h"

namespace gdn {

constexpr int kChunk = 64;
constexpr int kHD = 128;                 // Dk = Dv
constexpr int kSliceRows = 16;           // state rows per state-pass workgroup
constexpr int kSlices = kHD / kSliceRows;
constexpr float kLogGateFloor = -80.f;   // exp(-80) ~ 1.8e-35: a reset state

// Per (chunk, value head) record written by the chunk pass. Tb and P are
// stored as MFMA A-operand fragments: fragment f = 2 rb + kb holds rows
// 16 rb .. +15 and columns 32 kb .. +31, lane l of it the 8 values of row
// 16 rb + l%16, columns 32 kb + 8(l/16) .. +7 (16 bytes at 16 (64 f + l)), so
// that a wave loads its operand as one contiguous 1 KiB. Fragments (0, 1) and
// (1, 1) lie above the diagonal (all zero) and are neither written nor read.
constexpr int64_t kMatBytes = int64_t(kChunk) * kChunk * 2;
constexpr int64_t kRecTbHi = 0, kRecTbLo = kMatBytes, kRecPHi = 2 * kMatBytes, kRecPLo = 3 * kMatBytes;
// exp(l_i) and exp(l_C - l_i) per token (l_C = l of the chunk's last token).
constexpr int64_t kRecEl = 4 * kMatBytes, kRecEd = kRecEl + kChunk * 4;
constexpr int64_t kRecBytes = 4 * kMatBytes + 2 * kChunk * 4;

GDN_DEV int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

__host__ __device__ inline int64_t records_offset(int N) { return ((int64_t(N) + 1) * 4 + 255) & ~int64_t(255); }
__host__ __device__ inline int64_t chunks_bound(int64_t T, int N) { return T / kChunk + N + 1; }

GDN_DEV f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

GDN_DEV uint16_t bf16_bits(float x) { return f32_to_bf16_bits(x); }

// Split x into a bf16 high part and the bf16 of the residual.
GDN_DEV void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
    hi = bf16_bits(x);
    lo = bf16_bits(x - bf16_bits_to_f32(hi));
}

// Two values split at once (the same bits as split_bf16 on each): one
// v_cvt_pk_bf16_f32 for both high parts and one for both residuals, a in
// the low half of each dword. A lone wave issues a vector instruction only
// every ~9 cycles on this GPU (two waves per SIMD: ~4.7), so on the state
// recurrence's chain every instruction saved is time saved.
GDN_DEV void split_bf16x2(float a, float b, uint32_t& hi, uint32_t& lo) {
    hi = pack_bf16x2(a, b);
    lo = pack_bf16x2(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

GDN_DEV uint2 pack4(const uint16_t (&x)[4]) {
    return uint2{uint32_t(x[0]) | (uint32_t(x[1]) << 16), uint32_t(x[2]) | (uint32_t(x[3]) << 16)};
}

GDN_DEV bf16x8 load8(const uint16_t* p) { return *reinterpret_cast<const bf16x8*>(p); }

// Eight consecutive float32 inputs as bf16 high parts and bf16 residuals.
GDN_DEV void load_split8(const float* p, u16x8& hi, u16x8& lo) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint16_t h, o;
        split_bf16(x[j], h, o);
        hi[j] = h;
        lo[j] = o;
    }
}

// A value loaded as its raw bits (the low 16 for bf16 and f16) as float.
GDN_DEV float raw_to_f32(uint32_t raw, int dtype) {
    if (dtype == GDN_F32) return __uint_as_float(raw);
    return dtype == GDN_BF16 ? bf16_bits_to_f32(uint16_t(raw)) : f16_bits_to_f32(uint16_t(raw));
}

GDN_DEV bf16x8 zero8() {
    bf16x8 z;
#pragma unroll
    for (int j = 0; j < 8; ++j) z[j] = __bf16(0.f);
    return z;
}

// ---------------------------------------------------------------------------
// run / chunk bookkeeping
// ---------------------------------------------------------------------------

// Packed runs: chunk_off[i] = index of run i's first chunk; chunk_off[N] =
// chunk count.
__global__ void chunk_offsets_kernel(const int32_t* __restrict__ cu, int N,
                                     int32_t* __restrict__ chunk_off) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    int32_t off = 0;
    for (int i = 0; i < N; ++i) {
        chunk_off[i] = off;
        off += int32_t((int64_t(cu[i + 1]) - cu[i] + kChunk - 1) / kChunk);
    }
    chunk_off[N] = off;
}

// Where the runs and their chunks lie: packed runs (cu) with the chunk
// offsets chunk_offsets_kernel wrote, or N runs of L_uniform tokens, cpr
// chunks each (no offsets needed, and no launch for them).
struct RunLayout {
    const int32_t* cu;
    const int32_t* chunk_off;  // null for uniform runs
    int64_t L_uniform;
    int N, cpr;

    GDN_DEV int total() const { return chunk_off ? chunk_off[N] : N * cpr; }
    GDN_DEV int first(int run) const { return chunk_off ? chunk_off[run] : run * cpr; }
    GDN_DEV int run_of(int g) const { return chunk_off ? find_run(chunk_off, N, g) : g / cpr; }
    GDN_DEV int64_t start(int run) const { return cu ? cu[run] : run * L_uniform; }
    GDN_DEV int64_t end(int run) const { return cu ? cu[run + 1] : (run + 1) * L_uniform; }
};

struct ChunkPos {
    int run;
    int64_t t0;  // first token
    int len;     // tokens in the chunk (1..64)
};

GDN_DEV ChunkPos locate_chunk(const RunLayout& rl, int g) {
    const int run = rl.run_of(g);
    const int64_t t0 = rl.start(run) + int64_t(g - rl.first(run)) * kChunk;
    const int64_t rest = rl.end(run) - t0;
    return {run, t0, int(rest < kChunk ? rest : kChunk)};
}

// ---------------------------------------------------------------------------
// chunk pass
// ---------------------------------------------------------------------------

constexpr int kKS = kHD + 8;    // bf16 row stride of the K/Q tiles
constexpr int kFS = kChunk + 1; // float row stride of the A/T/P tiles
constexpr float kLog2e = 1.4426950408889634f;

// Stores a lower-triangular 64 x 64 float32 tile held in LDS (row stride
// kFS) as bf16 hi + lo fragments (layout above), 16 bytes per lane, by
// `nthreads` threads numbered `t`. With col_scale (T diag(beta)): the
// diagonal is taken as 1 and column j is scaled by col_scale[j]; without it,
// entries above the diagonal are zero.
GDN_DEV void store_fragments(const float* M, uint16_t* hi_out, uint16_t* lo_out,
                             const float* col_scale, int t, int nthreads) {
    for (int item = t; item < 6 * 64; item += nthreads) {
        const int fi = item >> 6, ln = item & 63;
        const int f = fi < 2 ? 2 * fi : fi + 2;  // skip fragments 1 and 3
        const int i = 16 * (f >> 1) + (ln & 15), j0 = 32 * (f & 1) + 8 * (ln >> 4);
        u16x8 h, o;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int j = j0 + jj;
            float x = i > j ? M[i * kFS + j] : 0.f;
            if (col_scale) x = (i == j ? 1.f : x) * col_scale[j];
            else if (i == j) x = M[i * kFS + j];
            uint16_t a, b;
            split_bf16(x, a, b);
            h[jj] = a;
            o[jj] = b;
        }
        *reinterpret_cast<u16x8*>(hi_out + (64 * f + ln) * 8) = h;
        *reinterpret_cast<u16x8*>(lo_out + (64 * f + ln) * 8) = o;
    }
}

// The four diagonal blocks of T = (I + A)^-1 (A strictly lower triangular),
// by one wave: lane (b = l/16, n = l%16) solves (I + A_bb) x = e_n by
// column-oriented forward substitution and writes x as column n of T_bb.
GDN_DEV void diag_inverse(const float* As, float* Ts, int l) {
    const int b = l >> 4, n = l & 15;
    const float* Ab = As + 16 * b * kFS + 16 * b;
    float s[16], x[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) s[m] = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        x[k] = k == n ? 1.f : (k > n ? -s[k] : 0.f);
#pragma unroll
        for (int m = k + 1; m < 16; ++m) s[m] += Ab[m * kFS + k] * x[k];
    }
    float* Tb = Ts + 16 * b * kFS + 16 * b;
#pragma unroll
    for (int m = 0; m < 16; ++m) Tb[m * kFS + n] = x[m];
}

// acc += X Y for 16 x 16 float32 blocks in LDS (row stride kFS), on
// v_mfma_f32_16x16x4f32 (lane l: X[l%16][4kb + l/16], Y[4kb + l/16][l%16];
// acc[i] = (XY)[4(l/16) + i][l%16]).
GDN_DEV f32x4 mma_f32(const float* X, const float* Y, f32x4 acc, int l) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        const float a = X[(l & 15) * kFS + 4 * kb + (l >> 4)];
        const float b = Y[(4 * kb + (l >> 4)) * kFS + (l & 15)];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
    }
    return acc;
}

GDN_DEV void put_block(float* O, f32x4 v, float scale, int l) {
#pragma unroll
    for (int i = 0; i < 4; ++i) O[(4 * (l >> 4) + i) * kFS + (l & 15)] = scale * v[i];
}

GDN_DEV float* blk(float* M, int bi, int bj) { return M + 16 * bi * kFS + 16 * bj; }
GDN_DEV const float* blk(const float* M, int bi, int bj) { return M + 16 * bi * kFS + 16 * bj; }

// Off-diagonal blocks of T from its diagonal blocks, by recursive doubling
// over 16 x 16 blocks (T_ij = -T_ii sum_k A_ik T_kj): first the two 32 x 32
// diagonal halves, then T[2:4, 0:2] = -T[2:4, 2:4] (A[2:4, 0:2] T[0:2, 0:2]).
// The intermediate product X_ij is kept in A's (all-zero, unread) block
// (j, i) above the diagonal. Ends with a barrier.
GDN_DEV void offdiag_inverse(float* As, float* Ts, int w, int l) {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    if (w < 2) {  // T_10 (wave 0), T_32 (wave 1)
        const int j = 2 * w, i = j + 1;
        put_block(blk(As, j, i), mma_f32(blk(As, i, j), blk(Ts, j, j), zero, l), 1.f, l);
        put_block(blk(Ts, i, j), mma_f32(blk(Ts, i, i), blk(As, j, i), zero, l), -1.f, l);
    }
    __syncthreads();
    const int i = 2 + (w >> 1), j = w & 1;  // one block of T[2:4, 0:2] per wave
    f32x4 x = zero;
    for (int k = j; k < 2; ++k) x = mma_f32(blk(As, i, k), blk(Ts, k, j), x, l);
    put_block(blk(As, j, i), x, 1.f, l);
    __syncthreads();
    f32x4 t = zero;
    for (int k = 2; k <= i; ++k) t = mma_f32(blk(Ts, i, k), blk(As, j, k), t, l);
    put_block(blk(Ts, i, j), t, -1.f, l);
    __syncthreads();
}

// One workgroup per (chunk, value head), or with float32 input per (chunk,
// two value heads of one key head). K K^T and K Q^T depend only on the key
// head; with bf16 input recomputing them per value head (32 MFMAs per wave)
// keeps each workgroup within the 128 registers that let four share a CU
// (holding them for a second head spills), while the float32 products
// (three MFMAs each, from split operands) are worth sharing at two
// workgroups per CU. Workgroup ids go round-robin over the 8 XCDs, so the
// workgroups of one (chunk, key head) take ids 8 apart: same XCD,
// dispatched together, so all but the first read that chunk's K and Q from
// the XCD's L2.
//
// The raw projection rows and conv parameters of the fused chunk pass, which
// computes q, k and v itself (the prefill front-end, linear_attention.py:61-79,
// 103-113) and leaves them for the state pass.
struct ConvIn {
    const uint16_t* qkv;      // (T, qs) bf16: the q, k and v channels of each token
    int64_t qs;               // qkv row stride (elements)
    const void* cs_in;        // (N, K-1, C) conv states, in the kernel's conv dtype
    uint16_t* cs_out;         // (N, K-1, C) new conv states, bf16
    const float* w;           // (C, K) conv weights
    uint16_t *qo, *ko, *vo;   // (T, Hk, 128), (T, Hk, 128), (T, Hv, 128) bf16
};

// The inputs of the chunk pass: bf16 q and k, float32 q and k, or (fused)
// the raw projection rows and a conv state in bf16 or float32.
constexpr int kInBF16 = 0, kInF32 = 1, kInConvBF16 = 2, kInConvF32 = 3;

// Workgroup id -> (chunk-and-key-head item, first value head e0 of the
// key head's group): a workgroup takes kHeads consecutive value heads of one
// key head, which share the chunk's K K^T and K Q^T; ids go over 8 items,
// then over the head sets, then over the next 8 items.
template <int kHeads>
GDN_DEV void chunk_item(int id, int r, int& item, int& e0) {
    const int rh = r / kHeads;
    e0 = ((id >> 3) % rh) * kHeads;
    item = (id / (8 * rh)) * 8 + (id & 7);
}

// kInF32: q and k are float32, entering the MFMAs as bf16 high parts plus
// residuals (hi.hi + hi.lo + lo.hi), with two more LDS tiles for the
// residuals; kInBF16: bf16, used as they are. kInConv*: each workgroup runs
// the front-end for its chunk's q and k with the arithmetic of the tiled
// front-end kernel (conv, SiLU, the scaled RMS norm, the same bits): thread
// (group g: q or k, rows 8 rg .. 8 rg + 7, channels 8 seg .. 8 seg + 7) walks
// its rows with the previous three in registers (a run's first rows take
// them from its conv state) into the K / Q tiles; the first value head of
// each key head also stores q and k for the state pass (v: conv_v_block).
// `id` is the workgroup's index in chunk_item's order. The workgroup records
// kHeads value heads in turn from one set of products.
template <int kIn, int kHeads>
GDN_DEV void prefill_chunk_body(
    const void* __restrict__ q_in, const void* __restrict__ k_in, const void* __restrict__ ga,
    const void* __restrict__ gb, int gb_dtype, int64_t gate_stride, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, int gate_mode, RunLayout rl, char* __restrict__ records,
    int Hk, int Hv, ConvIn cv = {}, int id = -1) {
    constexpr bool kF32 = kIn == kInF32;
    constexpr bool kConv = kIn == kInConvBF16 || kIn == kInConvF32;
    constexpr int kConvDt = kIn == kInConvF32 ? GDN_F32 : GDN_BF16;
    // K/Q tiles first; once K K^T and K Q^T are in registers the same bytes
    // hold the A and T matrices.
    __shared__ __attribute__((aligned(16))) char smem[(kF32 ? 4 : 2) * kChunk * kKS * 2];
    __shared__ __attribute__((aligned(16))) float l2_sh[kChunk], beta_sh[kChunk];
    uint16_t* Ks = reinterpret_cast<uint16_t*>(smem);
    uint16_t* Qs = Ks + kChunk * kKS;
    uint16_t* Ks_lo = Qs + kChunk * kKS;  // kF32 only
    uint16_t* Qs_lo = Ks_lo + kChunk * kKS;
    float* As = reinterpret_cast<float*>(smem);
    float* Ts = As + kChunk * kFS;

    const int r = Hv / Hk;
    if (id < 0) id = blockIdx.x;
    int item, e0;  // (chunk, key head), first value head of the set
    chunk_item<kHeads>(id, r, item, e0);
    const int g = item / Hk, hk = item % Hk, hv0 = hk * r + e0;
    if (g >= rl.total()) return;
    const ChunkPos pos = locate_chunk(rl, g);
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    auto rec_of = [&](int h) { return records + (int64_t(g) * Hv + hv0 + h) * kRecBytes; };

    // The gate inputs of wave 0 (lane = token) go out first, as raw words
    // decoded where they are used, so that the gates' prefix sum does not
    // wait behind the K and Q loads.
    uint32_t ga_raw[kHeads] = {}, gb_raw[kHeads] = {};
    if (w == 0) {
        const int lc = l < pos.len ? l : pos.len - 1;
#pragma unroll
        for (int h = 0; h < kHeads; ++h) {
            const int64_t i = (pos.t0 + lc) * gate_stride + hv0 + h;
            ga_raw[h] = gate_mode == 1 || gb_dtype == GDN_F32 ? static_cast<const uint32_t*>(ga)[i]
                                                              : static_cast<const uint16_t*>(ga)[i];
            gb_raw[h] = gb_dtype == GDN_F32 ? static_cast<const uint32_t*>(gb)[i]
                                            : static_cast<const uint16_t*>(gb)[i];
        }
    }

    // K and Q of the chunk: every load issued before the first LDS store
    // (rows past the run are read clamped and stored as zero).
    u16x8 kv[4], qv[4], kvl[4], qvl[4];
    // fused: this thread's raw rows, the three before them and its weights
    const int cgrp = tid >> 7, crg = (tid >> 4) & 7, cseg = tid & 15;
    const int C = (2 * Hk + Hv) * kHD;
    uint4 raw[8];
    float win[3][8], wr[8][4];
    if constexpr (kConv) {
        const int64_t c0 = int64_t(cgrp * Hk + hk) * kHD + cseg * 8;
        const int64_t rs = rl.start(pos.run), last = rl.end(pos.run) - 1;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t t = pos.t0 + 8 * crg + i;
            raw[i] = *reinterpret_cast<const uint4*>(cv.qkv + (t < last ? t : last) * cv.qs + c0);
        }
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int64_t t = pos.t0 + 8 * crg - 3 + j;
            if (t >= rs)
                unpack8(*reinterpret_cast<const uint4*>(cv.qkv + (t < last ? t : last) * cv.qs + c0), win[j]);
            else  // row t - rs + 3 of the run's conv state
                load_state8<kConvDt>(cv.cs_in, (int64_t(pos.run) * 3 + (t - rs + 3)) * C + c0, win[j]);
        }
        load_conv_w8(cv.w, c0, wr);
    } else {
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int row = (tid + 256 * it) >> 4, seg = tid & 15;
            const int rc = row < pos.len ? row : pos.len - 1;
            const int64_t off = ((pos.t0 + rc) * Hk + hk) * kHD + seg * 8;
            if constexpr (kF32) {
                load_split8(static_cast<const float*>(k_in) + off, kv[it], kvl[it]);
                load_split8(static_cast<const float*>(q_in) + off, qv[it], qvl[it]);
            } else {
                kv[it] = *reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(k_in) + off);
                qv[it] = *reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(q_in) + off);
            }
        }
    }
    // Gates of value head hv0 + h (wave 0, lane = token): l2 = inclusive
    // prefix sum of log2 g (exp2 of differences gives the decays).
    auto gates = [&](int h) {
        const int hv = hv0 + h;
        char* rec = rec_of(h);
        float lg, beta;
        const float gbv = raw_to_f32(gb_raw[h], gb_dtype);
        if (gate_mode == 0) {
            lg = log_forget_gate(raw_to_f32(ga_raw[h], gb_dtype), A_log[hv], dt_bias[hv]);
            beta = beta_of(gbv, gb_dtype);
        } else {
            const float gv = __uint_as_float(ga_raw[h]);
            lg = gv > 0.f ? logf(gv) : kLogGateFloor;
            beta = gbv;
        }
        lg = l < pos.len ? fmaxf(lg, kLogGateFloor) * kLog2e : 0.f;
        beta = l < pos.len ? beta : 0.f;
#pragma unroll
        for (int off = 1; off < kChunk; off <<= 1) {
            const float y = __shfl_up(lg, off, kWave);
            if (l >= off) lg += y;
        }
        l2_sh[l] = lg;
        beta_sh[l] = beta;
        const float lC = __shfl(lg, kChunk - 1, kWave);
        reinterpret_cast<float*>(rec + kRecEl)[l] = exp2f(lg);
        reinterpret_cast<float*>(rec + kRecEd)[l] = exp2f(lC - lg);
    };
    if (w == 0) gates(0);
    if constexpr (kConv) {
        // conv, SiLU and the scaled norm of rows 8 crg .. 8 crg + 7 into the
        // tile; the first value head of the key head also stores them
        const float inv = 1.f / sqrtf(float(kHD));
        const float sc = cgrp == 0 ? round_bf16(inv * inv) : round_bf16(inv);
        uint16_t* tile = cgrp == 0 ? Qs : Ks;
        uint16_t* out = (cgrp == 0 ? cv.qo : cv.ko) + int64_t(hk) * kHD + cseg * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = 8 * crg + i;
            float x[8], o[8], n[8];
            unpack8(raw[i], x);
            conv_silu8(wr, win, x, o);
            rms_norm8(o, n);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = sc * n[e];
            const uint4 p = pack8(o);
            *reinterpret_cast<uint4*>(tile + row * kKS + cseg * 8) = row < pos.len ? p : make_uint4(0, 0, 0, 0);
            if (e0 == 0 && row < pos.len) *reinterpret_cast<uint4*>(out + (pos.t0 + row) * Hk * kHD) = p;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                win[0][j] = win[1][j];
                win[1][j] = win[2][j];
                win[2][j] = x[j];
            }
        }
    } else {
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int row = (tid + 256 * it) >> 4, seg = tid & 15;
            const u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
            *reinterpret_cast<u16x8*>(Ks + row * kKS + seg * 8) = row < pos.len ? kv[it] : z;
            *reinterpret_cast<u16x8*>(Qs + row * kKS + seg * 8) = row < pos.len ? qv[it] : z;
            if constexpr (kF32) {
                *reinterpret_cast<u16x8*>(Ks_lo + row * kKS + seg * 8) = row < pos.len ? kvl[it] : z;
                *reinterpret_cast<u16x8*>(Qs_lo + row * kKS + seg * 8) = row < pos.len ? qvl[it] : z;
            }
        }
    }
    __syncthreads();

    // K K^T and K Q^T: wave w owns key rows 16w..16w+15, all four column
    // tiles; kk[jt][ii] = k_i . k_j and kq[jt][ii] = k_i . q_j for
    // i = 16w + 4(l/16) + ii, j = 16jt + l%16.
    f32x4 kk[4], kq[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) kk[jt] = kq[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int lr = l & 15, lq = l >> 4, lg8 = 8 * lq;
#pragma unroll
    for (int s = 0; s < kHD / 32; ++s) {
        const bf16x8 ak = load8(Ks + (16 * w + lr) * kKS + 32 * s + lg8);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            kk[jt] = mfma16(ak, load8(Ks + (16 * jt + lr) * kKS + 32 * s + lg8), kk[jt]);
            kq[jt] = mfma16(ak, load8(Qs + (16 * jt + lr) * kKS + 32 * s + lg8), kq[jt]);
        }
    }
    if constexpr (kF32) {  // the residual products, summed apart and added once
        f32x4 kk2[4], kq2[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) kk2[jt] = kq2[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kHD / 32; ++s) {
            const bf16x8 ak = load8(Ks + (16 * w + lr) * kKS + 32 * s + lg8);
            const bf16x8 akl = load8(Ks_lo + (16 * w + lr) * kKS + 32 * s + lg8);
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                const int ro = (16 * jt + lr) * kKS + 32 * s + lg8;
                kk2[jt] = mfma16(ak, load8(Ks_lo + ro), kk2[jt]);
                kk2[jt] = mfma16(akl, load8(Ks + ro), kk2[jt]);
                kq2[jt] = mfma16(ak, load8(Qs_lo + ro), kq2[jt]);
                kq2[jt] = mfma16(akl, load8(Qs + ro), kq2[jt]);
            }
        }
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            kk[jt] += kk2[jt];
            kq[jt] += kq2[jt];
        }
    }
    __syncthreads();  // K/Q tiles are dead from here on

#pragma unroll
    for (int h = 0; h < kHeads; ++h) {
        if (h > 0) {
            __syncthreads();  // the previous head's readers of l2_sh, beta_sh, As and Ts are done
            if (w == 0) gates(h);
            __syncthreads();
        }
        char* rec = rec_of(h);
        // A (row i, column j) into LDS and P (query j, key i) straight from the
        // accumulators into its fragments: lane (l%16, l/16) of wave w holds keys
        // 16w + 4(l/16) .. +3 of query 16jt + l%16, which is half of the 16-byte
        // entry (query row l%16, keys 8g .. 8g+7) of fragment (jt, w/2), with
        // g = 2(w%2) + (l/16)/2, half (l/16)%2. Fragments above the diagonal
        // (jt < 2 <= w) are skipped.
        const float4 li = *reinterpret_cast<const float4*>(l2_sh + 16 * w + 4 * lq);
        const float4 bi = *reinterpret_cast<const float4*>(beta_sh + 16 * w + 4 * lq);
        const float l2i[4] = {li.x, li.y, li.z, li.w}, betai[4] = {bi.x, bi.y, bi.z, bi.w};
        uint16_t* p_hi = reinterpret_cast<uint16_t*>(rec + kRecPHi);
        uint16_t* p_lo = reinterpret_cast<uint16_t*>(rec + kRecPLo);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            const int j = 16 * jt + lr;
            const float l2j = l2_sh[j];
            uint16_t ph[4], pl[4];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int i = 16 * w + 4 * lq + ii;
                const float d = l2i[ii] - l2j;  // <= 0 for i >= j, >= 0 for i <= j
                const float dki = exp2f(i > j ? d : -d);
                As[i * kFS + j] = i > j ? betai[ii] * kk[jt][ii] * dki : 0.f;
                split_bf16(i <= j ? kq[jt][ii] * dki : 0.f, ph[ii], pl[ii]);
            }
            if (w < 2 || jt >= 2) {
                const int f = 2 * jt + (w >> 1), ln = 16 * (2 * (w & 1) + (lq >> 1)) + lr;
                const int off = (64 * f + ln) * 8 + 4 * (lq & 1);
                *reinterpret_cast<uint2*>(p_hi + off) = pack4(ph);
                *reinterpret_cast<uint2*>(p_lo + off) = pack4(pl);
            }
        }
        __syncthreads();
        if (w == 0) diag_inverse(As, Ts, l);  // T's diagonal blocks
        __syncthreads();
        offdiag_inverse(As, Ts, w, l);
        // Tb = T diag(beta), split into bf16 hi + lo.
        store_fragments(Ts, reinterpret_cast<uint16_t*>(rec + kRecTbHi),
                        reinterpret_cast<uint16_t*>(rec + kRecTbLo), beta_sh, tid, 256);
    }
}

// The fused chunk pass's v part, done by each chunk workgroup after its
// records: the front-end of chunk g's v channels of value head hv, for the
// state pass (SiLU(conv), no norm), thread (rows 4 rg .. 4 rg + 3, channels
// 8 seg ..). (Separate v workgroups interleaved with the chunk workgroups
// were slower: 84 against 64 us at T=4096, as they take the LDS-limited
// workgroup slots.) The workgroups of a run's last chunk also write the
// run's new conv state (row j: row len + j of concat(state, tokens)): the v
// channels of hv, and with the first value head the q and k channels of hk;
// 48 pieces of 8 channels a group.
template <int kConvDt>
GDN_DEV void conv_v_block(RunLayout rl, const ConvIn& cv, int item, int e, int Hk, int Hv) {
    const int r = Hv / Hk;
    const int g = item / Hk, hk = item % Hk, hv = hk * r + e;
    if (g >= rl.total()) return;
    const ChunkPos pos = locate_chunk(rl, g);
    const int tid = threadIdx.x;
    const int C = (2 * Hk + Hv) * kHD;
    float win[3][8], wr[8][4];
    const int vrg = tid >> 4, vseg = tid & 15;
    const int64_t c0 = int64_t(2 * Hk + hv) * kHD + vseg * 8;
    const int64_t rs = rl.start(pos.run), last = rl.end(pos.run) - 1;
    uint4 vraw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t t = pos.t0 + 4 * vrg + i;
        vraw[i] = *reinterpret_cast<const uint4*>(cv.qkv + (t < last ? t : last) * cv.qs + c0);
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int64_t t = pos.t0 + 4 * vrg - 3 + j;
        if (t >= rs)
            unpack8(*reinterpret_cast<const uint4*>(cv.qkv + (t < last ? t : last) * cv.qs + c0), win[j]);
        else
            load_state8<kConvDt>(cv.cs_in, (int64_t(pos.run) * 3 + (t - rs + 3)) * C + c0, win[j]);
    }
    load_conv_w8(cv.w, c0, wr);
    uint16_t* out = cv.vo + int64_t(hv) * kHD + vseg * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * vrg + i;
        float x[8], o[8];
        unpack8(vraw[i], x);
        conv_silu8(wr, win, x, o);
        if (row < pos.len) *reinterpret_cast<uint4*>(out + (pos.t0 + row) * Hv * kHD) = pack8(o);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            win[0][j] = win[1][j];
            win[1][j] = win[2][j];
            win[2][j] = x[j];
        }
    }
    if (pos.t0 + pos.len == rl.end(pos.run)) {  // the run's last chunk: its new conv state
        const int64_t len = rl.end(pos.run) - rs;
        const int grp = tid / 48, pc = tid % 48, j = pc / 16, sg = pc % 16;
        if (grp < 3 && (grp == 2 || e == 0)) {
            const int64_t ch = (grp == 2 ? int64_t(2 * Hk + hv) : int64_t(grp * Hk + hk)) * kHD + sg * 8;
            const int64_t idx = len + j;  // in concat(state, tokens)
            uint4 v;
            if (idx < 3) {
                float x[8];
                load_state8<kConvDt>(cv.cs_in, (int64_t(pos.run) * 3 + idx) * C + ch, x);
                v = pack8(x);
            } else {
                v = *reinterpret_cast<const uint4*>(cv.qkv + (rs + idx - 3) * cv.qs + ch);
            }
            *reinterpret_cast<uint4*>(cv.cs_out + (int64_t(pos.run) * 3 + j) * C + ch) = v;
        }
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void prefill_chunk_kernel(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ ga,
    const void* __restrict__ gb, int gb_dtype, int64_t gate_stride, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, int gate_mode, RunLayout rl, char* __restrict__ records,
    int Hk, int Hv) {
    prefill_chunk_body<kInBF16, 1>(q, k, ga, gb, gb_dtype, gate_stride, A_log, dt_bias, gate_mode, rl,
                                records, Hk, Hv);
}

template <int kHeads>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void prefill_chunk_f32_kernel(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ ga,
    const void* __restrict__ gb, int gb_dtype, int64_t gate_stride, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, int gate_mode, RunLayout rl, char* __restrict__ records,
    int Hk, int Hv) {
    prefill_chunk_body<kInF32, kHeads>(q, k, ga, gb, gb_dtype, gate_stride, A_log, dt_bias, gate_mode, rl,
                               records, Hk, Hv);
}

// The fused chunk pass: the front-end (bf16 projection rows, conv state in
// bf16 or float32) and the chunk pass in one launch; each workgroup ends
// with the v channels of its (chunk, value head).
template <int kConvDt>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void prefill_chunk_conv_kernel(
    const void* __restrict__ ga, const void* __restrict__ gb, int gb_dtype, int64_t gate_stride,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias, RunLayout rl,
    char* __restrict__ records, int Hk, int Hv, ConvIn cv) {
    prefill_chunk_body<kConvDt == GDN_F32 ? kInConvF32 : kInConvBF16, 1>(
        nullptr, nullptr, ga, gb, gb_dtype, gate_stride, A_log, dt_bias, 0, rl, records, Hk, Hv, cv);
    int item, e;
    chunk_item<1>(blockIdx.x, Hv / Hk, item, e);
    conv_v_block<kConvDt>(rl, cv, item, e, Hk, Hv);
}

// The new conv state of each empty run (no chunk writes it): its old state,
// rounded to bf16. One block per run.
template <int kConvDt>
__global__ __launch_bounds__(256) void conv_state_empty_runs_kernel(RunLayout rl, ConvIn cv, int C) {
    const int run = blockIdx.x;
    if (rl.end(run) != rl.start(run)) return;
    for (int64_t i = threadIdx.x * 8; i < 3 * int64_t(C); i += 256 * 8) {
        float x[8];
        load_state8<kConvDt>(cv.cs_in, int64_t(run) * 3 * C + i, x);
        *reinterpret_cast<uint4*>(cv.cs_out + int64_t(run) * 3 * C + i) = pack8(x);
    }
}

// ---------------------------------------------------------------------------
// state pass
// ---------------------------------------------------------------------------

constexpr int kSS = kHD + 8;     // bf16 row stride of the S operand tile
constexpr int kTS = kChunk + 8;  // bf16 row stride of token-minor operand tiles

typedef short v4s __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The state pass runs 8 waves per workgroup. Waves 0-3 carry the state
// recurrence (S K^T -> R -> Tb R -> state update) and touch only LDS and
// their accumulators. Waves 4-7 compute the output (Q S^T, P D, y) and fetch
// every chunk operand from global memory for both halves: those of the
// state waves (K, V, Tb, the decay factors) two chunks ahead into registers,
// then into LDS one chunk ahead, and their own Q rows, straight into MFMA
// A fragments two chunks ahead. Issuing the loads is what the state
// recurrence cannot afford (the vector-memory queue stalls the issuing
// wave); the output waves have slack. Both halves meet at the same three
// barriers per chunk. Output wave w fetches the rows state wave w consumes;
// Tb and P are lower triangular, so the waves of token rows 0-31
// (kUpper = false) fetch and multiply only their first 32 columns.
constexpr int kStateThreads = 512;

// Chunk operands of state wave w, fetched by output wave w. They pass
// through registers on the way to LDS, so each load covers whole rows (full
// cache lines): 16 lanes per 256-byte K row, 8 per 128-byte Tb row.
struct StagedOperands {
    bf16x8 ka[4];           // K row 16w + 4i + l/16, dk 8(l%16) .. +7
    bf16x8 qa[4];           // Q: wave w's A fragments (row 16w + l%16, dk 32i + 8(l/16) .. +7)
    bf16x8 tbh[2], tbl[2];  // Tb fragments (2w + s) (hi, lo): row 16w + l%16, tokens 32s + 8(l/16) .. +7
    u32x2 v;                // V (bf16) at token 16w + l/4, dv dv0 + 4(l%4) .. +3
    f32x4 e;                // words 32w + 4(l%8) .. +3 of the record's [exp(l) | exp(l_C - l)]
    bf16x8 kal[4], qal[4];  // float32 input only (see below)
    u32x2 vl;
};
// Float32 input: the fetch keeps the loaded floats as they are (their bits:
// K's 8 values in ka[i] (0-3) and kal[i] (4-7), Q's likewise in qa/qal, V's
// 4 in v (0-1) and vl (2-3)); the staging (Q: the projection) splits them
// into bf16 hi + lo.
// Splitting at the fetch would wait there for every load it issues, which
// undoes the prefetch.

// P fragments of output wave w (used from registers).
struct OutputOperands {
    bf16x8 pah[2], pal[2];  // P rows 16w + l%16 (hi, lo)
};

// Per-run constants of a state-pass workgroup.
struct StatePassCtx {
    const void* q;
    const void* k;
    const void* v;
    const char* records;
    int64_t rs, re, qk_stride;
    int c0, h, hk, Hv, dv0;

    GDN_DEV int64_t t0(int c) const { return rs + int64_t(c) * kChunk; }
    GDN_DEV int len(int c) const {
        const int64_t r = re - t0(c);
        return r < kChunk ? int(r) : kChunk;
    }
    GDN_DEV const char* rec(int c) const { return records + (int64_t(c0 + c) * Hv + h) * kRecBytes; }
};

// Every load is unconditional, from a token index clamped into the chunk: a
// divergent conditional load would make the compiler wait for all
// outstanding loads (the prefetch included), and consuming a loaded value
// here would do the same. Rows past the run then hold copies of the last
// token, which contribute nothing: their beta and log-decay are zero, so
// their columns of Tb and P and their rows of D vanish. Addresses are a
// uniform per-chunk base plus a 32-bit lane offset.
template <bool kUpper, bool kF32>
GDN_DEV void fetch_staged(StagedOperands& op, const StatePassCtx& cx, int c, int w, int l) {
    const int len = cx.len(c);
    const int64_t qk0 = cx.t0(c) * cx.qk_stride + cx.hk * kHD + 8 * (l & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tok = 16 * w + 4 * i + (l >> 4);
        const int tok_c = tok < len ? tok : len - 1;
        const uint32_t o = uint32_t(tok_c) * uint32_t(cx.qk_stride);
        if constexpr (kF32) {
            const float* src = static_cast<const float*>(cx.k) + qk0 + o;
            op.ka[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const f32x4*>(src));
            op.kal[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const f32x4*>(src + 4));
        } else {
            op.ka[i] = load8(static_cast<const uint16_t*>(cx.k) + qk0 + o);
        }
    }
    // Q: output wave w reads only its own 16 rows; they load straight into
    // its A fragments (no LDS; float32 input: the raw floats, split into hi +
    // lo by the projection).
    {
        const int qtok = 16 * w + (l & 15), qtok_c = qtok < len ? qtok : len - 1;
        const int64_t q0 = cx.t0(c) * cx.qk_stride + cx.hk * kHD + 8 * (l >> 4) +
                           uint32_t(qtok_c) * uint32_t(cx.qk_stride);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (kF32) {
                const float* src = static_cast<const float*>(cx.q) + q0 + 32 * i;
                op.qa[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const f32x4*>(src));
                op.qal[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const f32x4*>(src + 4));
            } else {
                op.qa[i] = load8(static_cast<const uint16_t*>(cx.q) + q0 + 32 * i);
            }
        }
    }
    const int tv = 16 * w + (l >> 2);
    const int tv_c = tv < len ? tv : len - 1;
    const int64_t vo = cx.t0(c) * cx.Hv * kHD + cx.h * kHD + cx.dv0 + 4 * (l & 3) +
                       uint32_t(tv_c) * uint32_t(cx.Hv * kHD);
    if constexpr (kF32) {
        const f32x4 v4 = *reinterpret_cast<const f32x4*>(static_cast<const float*>(cx.v) + vo);
        op.v = u32x2{__float_as_uint(v4[0]), __float_as_uint(v4[1])};
        op.vl = u32x2{__float_as_uint(v4[2]), __float_as_uint(v4[3])};
    } else {
        op.v = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(cx.v) + vo);
    }
    const char* rec = cx.rec(c);
    op.e = *reinterpret_cast<const f32x4*>(rec + kRecEl + 128 * w + 16 * (l & 7));
    const uint16_t* tb_hi = reinterpret_cast<const uint16_t*>(rec + kRecTbHi);
    const uint16_t* tb_lo = reinterpret_cast<const uint16_t*>(rec + kRecTbLo);
#pragma unroll
    for (int s = 0; s < (kUpper ? 2 : 1); ++s) {
        op.tbh[s] = load8(tb_hi + (64 * (2 * w + s) + l) * 8);
        op.tbl[s] = load8(tb_lo + (64 * (2 * w + s) + l) * 8);
    }
}

template <bool kUpper>
GDN_DEV void fetch_output(OutputOperands& op, const StatePassCtx& cx, int c, int w, int l) {
    const char* rec = cx.rec(c);
    const uint16_t* p_hi = reinterpret_cast<const uint16_t*>(rec + kRecPHi);
    const uint16_t* p_lo = reinterpret_cast<const uint16_t*>(rec + kRecPLo);
#pragma unroll
    for (int s = 0; s < (kUpper ? 2 : 1); ++s) {
        op.pah[s] = load8(p_hi + (64 * (2 * w + s) + l) * 8);
        op.pal[s] = load8(p_lo + (64 * (2 * w + s) + l) * 8);
    }
}

// kF32 (float32 q, k, v): K and V also keep their bf16 residuals (Q stays
// in the output waves' registers for either input).
template <bool kF32>
struct StatePassLds {
    uint16_t Ss_hi[kSliceRows * kSS], Ss_lo[kSliceRows * kSS];  // S[dv][dk]
    uint16_t Kr[2][kChunk * kHD];                                 // K[token][dk] (swizzled), two buffers
    uint16_t Tb_hi[kChunk * kTS], Tb_lo[kChunk * kTS];            // Tb[token][token]
    uint16_t Vs[kChunk * kSliceRows];                             // V[token][dv]
    uint16_t Rs_hi[kSliceRows * kTS], Rs_lo[kSliceRows * kTS];    // R[dv][token]
    uint16_t Ds_hi[kSliceRows * kTS], Ds_lo[kSliceRows * kTS];    // D[dv][token]
    uint16_t D2_hi[kSliceRows * kTS], D2_lo[kSliceRows * kTS];    // D''[dv][token]
    float ex[2 * kChunk];                                         // exp(l), exp(l_C - l)
    uint16_t Kr_lo[kF32 ? 2 : 1][kF32 ? kChunk * kHD : 8];        // residuals (float32 input)
    uint16_t Vs_lo[kF32 ? kChunk * kSliceRows : 8];
};

// The K tile is read three ways: whole rows (staging), 16 rows at one
// 16-byte granule (K as an MFMA operand) and 4-row x 32-byte blocks (the
// transposing read). Rows are unpadded and granule G of row r is stored at
// G ^ kswz(r), which keeps all three free of LDS bank conflicts: kswz is a
// bijection of r % 16, and its upper three bits (r%4, bit 3 of r) differ
// across the 8 rows one transposing read pass touches.
GDN_DEV int kswz(int r) { return (((r & 3) | ((r >> 1) & 4)) << 1) | ((r >> 2) & 1); }
GDN_DEV int kr_off(int r, int G) { return r * kHD + ((G ^ kswz(r)) << 3); }

// Output waves: staged operands into LDS, in the layouts the state waves
// read them with (and, for float32 input, their own Q rows).
// The 8 floats whose bits a and b hold (4 each) as bf16 hi + lo, split in
// pairs (split_bf16x2: the same bits as split_bf16 on each).
GDN_DEV void split8_bits(const bf16x8& a, const bf16x8& b, bf16x8& hi, bf16x8& lo) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const f32x4 fa = __builtin_bit_cast(f32x4, a), fb = __builtin_bit_cast(f32x4, b);
    u32x4 h, r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float x0 = j < 2 ? fa[2 * j] : fb[2 * j - 4], x1 = j < 2 ? fa[2 * j + 1] : fb[2 * j - 3];
        uint32_t hj, rj;
        split_bf16x2(x0, x1, hj, rj);
        h[j] = hj;
        r[j] = rj;
    }
    hi = __builtin_bit_cast(bf16x8, h);
    lo = __builtin_bit_cast(bf16x8, r);
}

template <bool kF32>
GDN_DEV void stage_k(const StagedOperands& op, StatePassLds<kF32>& sm, int buf, int w, int l) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int o = kr_off(16 * w + 4 * i + (l >> 4), l & 15);
        if constexpr (kF32) {
            bf16x8 hi, lo;
            split8_bits(op.ka[i], op.kal[i], hi, lo);
            *reinterpret_cast<bf16x8*>(sm.Kr[buf] + o) = hi;
            *reinterpret_cast<bf16x8*>(sm.Kr_lo[buf] + o) = lo;
        } else {
            *reinterpret_cast<bf16x8*>(sm.Kr[buf] + o) = op.ka[i];
        }
    }
}

template <bool kF32>
GDN_DEV void stage_v(const StagedOperands& op, StatePassLds<kF32>& sm, int w, int l) {
    const int o = (16 * w + (l >> 2)) * kSliceRows + 4 * (l & 3);
    if constexpr (kF32) {
        uint32_t h0, r0, h1, r1;
        split_bf16x2(__uint_as_float(op.v[0]), __uint_as_float(op.v[1]), h0, r0);
        split_bf16x2(__uint_as_float(op.vl[0]), __uint_as_float(op.vl[1]), h1, r1);
        *reinterpret_cast<u32x2*>(sm.Vs + o) = u32x2{h0, h1};
        *reinterpret_cast<u32x2*>(sm.Vs_lo + o) = u32x2{r0, r1};
    } else {
        *reinterpret_cast<u32x2*>(sm.Vs + o) = op.v;
    }
}

// Lanes 8-63 repeat lanes 0-7 for the decay words (same words, same values):
// an unconditional store keeps the operand registers out of any branch.
template <bool kUpper, bool kF32>
GDN_DEV void stage_tb_e(const StagedOperands& op, StatePassLds<kF32>& sm, int w, int l) {
    const int row = (16 * w + (l & 15)) * kTS + 8 * (l >> 4);
#pragma unroll
    for (int s = 0; s < (kUpper ? 2 : 1); ++s) {
        *reinterpret_cast<bf16x8*>(sm.Tb_hi + row + 32 * s) = op.tbh[s];
        *reinterpret_cast<bf16x8*>(sm.Tb_lo + row + 32 * s) = op.tbl[s];
    }
    *reinterpret_cast<f32x4*>(sm.ex + 32 * w + 4 * (l & 7)) = op.e;
}

// State waves, chunk part 1: the S operand (hi + lo) into LDS.
template <bool kF32>
GDN_DEV void state_stage(const f32x4 (&acc)[2], StatePassLds<kF32>& sm, int w, int l) {
    const int lr = l & 15, lq = l >> 4;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int dk = 32 * w + 16 * t + 4 * lq;
        uint2 hi, lo;
        split_bf16x2(acc[t][0], acc[t][1], hi.x, lo.x);
        split_bf16x2(acc[t][2], acc[t][3], hi.y, lo.y);
        *reinterpret_cast<uint2*>(sm.Ss_hi + lr * kSS + dk) = hi;
        *reinterpret_cast<uint2*>(sm.Ss_lo + lr * kSS + dk) = lo;
    }
}

// State waves, part 2 (between the staging and R barriers):
// R^T = V^T - S K^T diag(exp l), lane (dv = 4(l/16) + i, token = 16w + l%16).
template <bool kF32>
GDN_DEV void state_residual(const StatePassLds<kF32>& sm, StatePassLds<kF32>& smw, int buf, int w, int l) {
    const int lr = l & 15, lq = l >> 4, lg8 = 8 * lq;
    const int tok = 16 * w + lr;
    f32x4 xk = {0.f, 0.f, 0.f, 0.f}, xk2 = xk;
#pragma unroll
    for (int s = 0; s < kHD / 32; ++s) {
        const int ko = kr_off(tok, 4 * s + lq);
        const bf16x8 kb = load8(sm.Kr[buf] + ko);
        const bf16x8 sh = load8(sm.Ss_hi + lr * kSS + 32 * s + lg8);
        xk = mfma16(sh, kb, xk);
        xk2 = mfma16(load8(sm.Ss_lo + lr * kSS + 32 * s + lg8), kb, xk2);
        if constexpr (kF32) xk2 = mfma16(sh, load8(sm.Kr_lo[buf] + ko), xk2);
    }
    xk += xk2;
    const float el = sm.ex[tok];
    const u32x2 vv = *reinterpret_cast<const u32x2*>(sm.Vs + tok * kSliceRows + 4 * lq);
    float v[4] = {__uint_as_float(vv[0] << 16), __uint_as_float(vv[0] & 0xffff0000u),
                  __uint_as_float(vv[1] << 16), __uint_as_float(vv[1] & 0xffff0000u)};
    if constexpr (kF32) {  // V = hi + residual (exact to ~16 significant bits)
        const u32x2 vr = *reinterpret_cast<const u32x2*>(sm.Vs_lo + tok * kSliceRows + 4 * lq);
        v[0] += __uint_as_float(vr[0] << 16);
        v[1] += __uint_as_float(vr[0] & 0xffff0000u);
        v[2] += __uint_as_float(vr[1] << 16);
        v[3] += __uint_as_float(vr[1] & 0xffff0000u);
    }
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
        uint32_t hi, lo;
        split_bf16x2(v[i] - el * xk[i], v[i + 1] - el * xk[i + 1], hi, lo);
        smw.Rs_hi[(4 * lq + i) * kTS + tok] = uint16_t(hi);
        smw.Rs_lo[(4 * lq + i) * kTS + tok] = uint16_t(lo);
        smw.Rs_hi[(4 * lq + i + 1) * kTS + tok] = uint16_t(hi >> 16);
        smw.Rs_lo[(4 * lq + i + 1) * kTS + tok] = uint16_t(lo >> 16);
    }
}

// State waves, part 3 (between the R and D barriers): D = Tb R, stored as
// D (hi + lo, for Y) and D'' = exp(l_C - l) D (hi + lo, for the update).
template <bool kUpper, bool kF32>
GDN_DEV void state_delta(StatePassLds<kF32>& sm, int w, int l) {
    const int lr = l & 15, lq = l >> 4, lg8 = 8 * lq;
    const int row = (16 * w + lr) * kTS + lg8;
    f32x4 d = {0.f, 0.f, 0.f, 0.f}, d2 = d;
#pragma unroll
    for (int s = 0; s < (kUpper ? 2 : 1); ++s) {
        const bf16x8 th = load8(sm.Tb_hi + row + 32 * s);
        const bf16x8 tl = load8(sm.Tb_lo + row + 32 * s);
        const bf16x8 bh = load8(sm.Rs_hi + lr * kTS + 32 * s + lg8);
        const bf16x8 bl = load8(sm.Rs_lo + lr * kTS + 32 * s + lg8);
        d = mfma16(th, bh, d);
        d2 = mfma16(th, bl, d2);
        d2 = mfma16(tl, bh, d2);
    }
    d += d2;
    const int tok0 = 16 * w + 4 * lq;
    const float4 ed = *reinterpret_cast<const float4*>(sm.ex + kChunk + tok0);
    const float e4[4] = {ed.x, ed.y, ed.z, ed.w};
    uint2 dh, dl, hi, lo;
    split_bf16x2(d[0], d[1], dh.x, dl.x);
    split_bf16x2(d[2], d[3], dh.y, dl.y);
    split_bf16x2(e4[0] * d[0], e4[1] * d[1], hi.x, lo.x);
    split_bf16x2(e4[2] * d[2], e4[3] * d[3], hi.y, lo.y);
    *reinterpret_cast<uint2*>(sm.Ds_hi + lr * kTS + tok0) = dh;
    *reinterpret_cast<uint2*>(sm.Ds_lo + lr * kTS + tok0) = dl;
    *reinterpret_cast<uint2*>(sm.D2_hi + lr * kTS + tok0) = hi;
    *reinterpret_cast<uint2*>(sm.D2_lo + lr * kTS + tok0) = lo;
}

// State waves, part 4 (after the D barrier): S^T <- exp(l_C) S^T + K^T D''.
// The K^T operand is read from the K tile with the transposing LDS read:
// within each 16-lane group, lane i of a ds_read_b64_tr_b16 receives element
// i%4 of source lane i/4 + 4k (k = 0..3); source lane s of group g points at
// K[8g + 4h + s/4][dk0 + 4(s%4)] for the tokens 8g + 4h .. +3.
template <bool kF32>
GDN_DEV void state_update(f32x4 (&acc)[2], const StatePassLds<kF32>& sm, int buf, float eC, int w,
                          int l) {
    const int g = l >> 4, sl = l & 15, lr = sl, lg8 = 8 * g;
    const uint16_t* kr = sm.Kr[buf];
    const uint16_t* krl = sm.Kr_lo[kF32 ? buf : 0];
    auto kt_operand = [&](const uint16_t* tile, int s, int dk0) {
        v4s parts[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int r = 32 * s + 8 * g + 4 * hh + (sl >> 2);
            const uint16_t* src = tile + kr_off(r, (dk0 >> 3) + ((sl & 3) >> 1)) + 4 * (sl & 1);
            parts[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4s*)(src));
        }
        return __builtin_bit_cast(bf16x8, __builtin_shufflevector(parts[0], parts[1], 0, 1, 2, 3, 4, 5, 6, 7));
    };
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        acc[t] *= eC;
        f32x4 lo_acc = {0.f, 0.f, 0.f, 0.f};
        const int dk0 = 32 * w + 16 * t;
#pragma unroll
        for (int s = 0; s < kChunk / 32; ++s) {
            const bf16x8 a = kt_operand(kr, s, dk0);
            const bf16x8 dh = load8(sm.D2_hi + lr * kTS + 32 * s + lg8);
            acc[t] = mfma16(a, dh, acc[t]);
            lo_acc = mfma16(a, load8(sm.D2_lo + lr * kTS + 32 * s + lg8), lo_acc);
            if constexpr (kF32) lo_acc = mfma16(kt_operand(krl, s, dk0), dh, lo_acc);
        }
        acc[t] += lo_acc;
    }
}

// Output waves, part 1 (between the staging and R barriers): exp(l) Q S^T,
// Q from the wave's registers (the chunk's operands).
template <bool kF32>
GDN_DEV f32x4 output_project(const StagedOperands& op, const StatePassLds<kF32>& sm, int w, int l) {
    const int lr = l & 15, lq = l >> 4, lg8 = 8 * lq;
    f32x4 xq = {0.f, 0.f, 0.f, 0.f}, xq2 = xq;
#pragma unroll
    for (int s = 0; s < kHD / 32; ++s) {
        bf16x8 qa = op.qa[s], ql;
        if constexpr (kF32) split8_bits(op.qa[s], op.qal[s], qa, ql);
        const bf16x8 sh = load8(sm.Ss_hi + lr * kSS + 32 * s + lg8);
        xq = mfma16(qa, sh, xq);
        xq2 = mfma16(qa, load8(sm.Ss_lo + lr * kSS + 32 * s + lg8), xq2);
        if constexpr (kF32) xq2 = mfma16(ql, sh, xq2);
    }
    xq += xq2;
    const float4 el = *reinterpret_cast<const float4*>(sm.ex + 16 * w + 4 * lq);
    xq[0] *= el.x;
    xq[1] *= el.y;
    xq[2] *= el.z;
    xq[3] *= el.w;
    return xq;
}

// Output waves, part 2 (after the D barrier): y = exp(l) Q S^T + P D.
template <class Y, bool kUpper, bool kF32>
GDN_DEV void output_store(const OutputOperands& op, f32x4 yacc, const StatePassLds<kF32>& sm,
                          const StatePassCtx& cx, int c, typename Y::storage* __restrict__ y, int w,
                          int l) {
    const int lr = l & 15, lq = l >> 4, lg8 = 8 * lq;
    f32x4 y2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < (kUpper ? 2 : 1); ++s) {
        const bf16x8 bh = load8(sm.Ds_hi + lr * kTS + 32 * s + lg8);
        const bf16x8 bl = load8(sm.Ds_lo + lr * kTS + 32 * s + lg8);
        yacc = mfma16(op.pah[s], bh, yacc);
        y2 = mfma16(op.pah[s], bl, y2);
        y2 = mfma16(op.pal[s], bh, y2);
    }
    yacc += y2;
    // Stores through a buffer resource that ends at the chunk's last token:
    // rows past the run fall outside it and the hardware drops them, so the
    // loop has no branch here (a branch lets the compiler sink the next
    // chunk's prefetch below it and wait for every outstanding load).
    using St = typename Y::storage;
    const int len = cx.len(c);
    const auto yr = __builtin_amdgcn_make_buffer_rsrc(y + cx.t0(c) * cx.Hv * kHD, 0,
                                                      len * cx.Hv * kHD * int(sizeof(St)), 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tok = 16 * w + 4 * lq + i;
        const int off = ((tok * cx.Hv + cx.h) * kHD + cx.dv0 + lr) * int(sizeof(St));
        if constexpr (Y::code == GDN_F32) {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yacc[i]), yr, off, 0, 0);
        } else if constexpr (Y::code == GDN_BF16) {
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(yacc[i]), yr, off, 0, 0);
        } else {
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_f16_bits(yacc[i]), yr, off, 0, 0);
        }
    }
}

// Chunk c: [S] B1 [R | Q S^T] B2 [D | Q, K, V(c+1), fetch c+2] B3
// [update | Tb(c+1), y]. Both loops are straight-line code (wave-uniform
// roles), so the compiler's waits for loaded operands are exact and never
// cover a later prefetch; both steps of the unrolled body are unconditional
// (an odd last chunk runs after the loop), because a conditional second step
// lets the compiler sink the first step's prefetch (invariant loads) to just
// before its use. Chunk indices past the run repeat its last chunk, so every
// fetch is unconditional.
template <bool kUpper, bool kF32>
GDN_DEV void state_loop(int nch, StatePassLds<kF32>& sm, f32x4 (&acc)[2], int w, int l) {
    auto step = [&](int buf) {
        state_stage(acc, sm, w, l);
        __syncthreads();
        state_residual(sm, sm, buf, w, l);
        const float eC = sm.ex[kChunk - 1];  // read before the next chunk restages it
        __syncthreads();
        state_delta<kUpper>(sm, w, l);
        __syncthreads();
        state_update(acc, sm, buf, eC, w, l);
    };
    int c = 0;
    for (; c + 1 < nch; c += 2) {
        step(0);
        step(1);
    }
    if (c < nch) step(0);
}

// Float32 input (operands with their residuals): chunk c + 2's operands
// fetched at step c, its P fragments one chunk ahead.
template <class Y, bool kUpper, bool kF32>
GDN_DEV void output_loop_2ahead(const StatePassCtx& cx, int nch, StatePassLds<kF32>& sm,
                         typename Y::storage* __restrict__ y, int w, int l) {
    const int last = nch - 1;
    StagedOperands ga, gb;
    OutputOperands oa, ob;
    // gn: staged operands of chunk c + 1 (in registers), gf: chunk c's (its
    // Q fragments are read first), then receives chunk c + 2
    auto step = [&](int c, int buf, const OutputOperands& oc, OutputOperands& on,
                    const StagedOperands& gn, StagedOperands& gf) {
        __syncthreads();
        const f32x4 yacc = output_project(gf, sm, w, l);  // gf still holds chunk c
        fetch_output<kUpper>(on, cx, c + 1 < last ? c + 1 : last, w, l);
        __builtin_amdgcn_sched_barrier(0);  // the prefetches stay where they are issued
        __syncthreads();
        stage_k(gn, sm, buf ^ 1, w, l);
        stage_v(gn, sm, w, l);
        fetch_staged<kUpper, kF32>(gf, cx, c + 2 < last ? c + 2 : last, w, l);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        stage_tb_e<kUpper>(gn, sm, w, l);
        output_store<Y, kUpper>(oc, yacc, sm, cx, c, y, w, l);
    };
    // chunk 0 into LDS; chunk 1 (or 0 again) into registers
    fetch_staged<kUpper, kF32>(gb, cx, 0, w, l);
    fetch_staged<kUpper, kF32>(ga, cx, 1 < last ? 1 : last, w, l);
    fetch_output<kUpper>(oa, cx, 0, w, l);
    stage_k(gb, sm, 0, w, l);
    stage_v(gb, sm, w, l);
    stage_tb_e<kUpper>(gb, sm, w, l);
    int c = 0;
    for (; c + 1 < nch; c += 2) {
        step(c, 0, oa, ob, ga, gb);
        step(c + 1, 1, ob, oa, gb, ga);
    }
    if (c < nch) step(c, 0, oa, ob, ga, gb);
}

// bf16 input: the operand loads are issued three chunks ahead and the P
// fragments two (at two chunks, the stores into LDS of the next chunk's
// operands waited for loads issued a whole step before: the phase between
// the second and third barrier is the step's longest). Chunk c's operands
// live in slot c % 3 of the ring, its P fragments in slot c % 3 of theirs.
template <class Y, bool kUpper, bool kF32>
GDN_DEV void output_loop_3ahead(const StatePassCtx& cx, int nch, StatePassLds<kF32>& sm,
                                typename Y::storage* __restrict__ y, int w, int l) {
    const int last = nch - 1;
    const auto at = [&](int c) { return c < last ? c : last; };
    StagedOperands g0, g1, g2;
    OutputOperands p0, p1, p2;
    // step c: cur holds chunk c (its Q read, then refilled with chunk c + 3),
    // nxt chunk c + 1 (staged into LDS); pc chunk c's P, pf receives c + 2's
    auto step = [&](int c, StagedOperands& cur, const StagedOperands& nxt, const OutputOperands& pc,
                    OutputOperands& pf) {
        __syncthreads();
        const f32x4 yacc = output_project(cur, sm, w, l);
        fetch_output<kUpper>(pf, cx, at(c + 2), w, l);
        __builtin_amdgcn_sched_barrier(0);  // the prefetches stay where they are issued
        __syncthreads();
        stage_k(nxt, sm, (c + 1) & 1, w, l);
        stage_v(nxt, sm, w, l);
        fetch_staged<kUpper, kF32>(cur, cx, at(c + 3), w, l);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        stage_tb_e<kUpper>(nxt, sm, w, l);
        output_store<Y, kUpper>(pc, yacc, sm, cx, c, y, w, l);
    };
    fetch_staged<kUpper, kF32>(g0, cx, 0, w, l);
    fetch_staged<kUpper, kF32>(g1, cx, at(1), w, l);
    fetch_staged<kUpper, kF32>(g2, cx, at(2), w, l);
    fetch_output<kUpper>(p0, cx, 0, w, l);
    fetch_output<kUpper>(p1, cx, at(1), w, l);
    stage_k(g0, sm, 0, w, l);
    stage_v(g0, sm, w, l);
    stage_tb_e<kUpper>(g0, sm, w, l);
    int c = 0;
    for (; c + 2 < nch; c += 3) {
        step(c, g0, g1, p0, p2);
        step(c + 1, g1, g2, p1, p0);
        step(c + 2, g2, g0, p2, p1);
    }
    if (c < nch) step(c, g0, g1, p0, p2);
    if (c + 1 < nch) step(c + 1, g1, g2, p1, p0);
}

template <class Y, bool kF32>
__global__ __launch_bounds__(kStateThreads) void prefill_state_kernel(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const float* __restrict__ state_in, float* __restrict__ state_out,
    typename Y::storage* __restrict__ y, RunLayout rl, const char* __restrict__ records, int Hk,
    int Hv) {
    __shared__ __attribute__((aligned(16))) StatePassLds<kF32> sm;

    // Work mapping: the 8 slices of one (run, head) share its K/Q and chunk
    // records, so they are placed on one XCD (workgroups go round-robin over
    // the 8 XCDs) when the head count allows it.
    const int R = rl.N * Hv;
    const int id = blockIdx.x;
    int hr, slice;
    if (R % 8 == 0) {
        const int xcd = id % 8, j = id / 8;
        hr = (j / 8) * 8 + xcd;
        slice = j % 8;
    } else {
        hr = id / kSlices;
        slice = id % kSlices;
    }
    const int run = hr / Hv, h = hr % Hv;
    const int tid = threadIdx.x;
    // wave-uniform (scalar) so that the wave roles take scalar branches
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool state_wave = wave < 4;
    const int w = wave & 3, l = tid & 63, lq = l >> 4, lr = l & 15;

    StatePassCtx cx;
    cx.q = q;
    cx.k = k;
    cx.v = v;
    cx.records = records;
    cx.rs = rl.start(run);
    cx.re = rl.end(run);
    cx.qk_stride = int64_t(Hk) * kHD;
    cx.c0 = rl.first(run);
    cx.h = h;
    cx.hk = h / (Hv / Hk);
    cx.Hv = Hv;
    cx.dv0 = slice * kSliceRows;
    const int nch = rl.first(run + 1) - cx.c0;

    if (state_wave) {
        // S^T in accumulators: acc[t][i] = S^T[dk = 32w + 16t + 4(l/16) + i][dv = dv0 + l%16].
        f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        const int64_t sbase = ((int64_t(run) * Hv + h) * kHD + cx.dv0 + lr) * kHD;
        if (state_in) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float4 s4 = *reinterpret_cast<const float4*>(state_in + sbase + 32 * w + 16 * t + 4 * lq);
                acc[t] = f32x4{s4.x, s4.y, s4.z, s4.w};
            }
        }
        if (nch > 0) {
            if (w >= 2) state_loop<true>(nch, sm, acc, w, l);
            else state_loop<false>(nch, sm, acc, w, l);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int dk = 32 * w + 16 * t + 4 * lq;
            *reinterpret_cast<float4*>(state_out + sbase + dk) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
        }
    } else if (nch > 0) {
        if constexpr (kF32) {
            if (w >= 2) output_loop_2ahead<Y, true>(cx, nch, sm, y, w, l);
            else output_loop_2ahead<Y, false>(cx, nch, sm, y, w, l);
        } else {
            if (w >= 2) output_loop_3ahead<Y, true>(cx, nch, sm, y, w, l);
            else output_loop_3ahead<Y, false>(cx, nch, sm, y, w, l);
        }
    }
}

}  // namespace gdn

using namespace gdn;

extern "C" int64_t gdn_prefill_workspace_size(int N, int64_t T_total, int Hk, int Hv, int Dk, int Dv) {
    if (N <= 0 || T_total < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return fail(GDN_EINVAL, "gdn_prefill_workspace_size: bad sizes");
    if (Dk != kHD || Dv != kHD) return fail(GDN_EUNSUPPORTED, "gdn_prefill_workspace_size: specialised for Dk=Dv=128");
    return records_offset(N) + chunks_bound(T_total, N) * Hv * kRecBytes;
}

extern "C" int gdn_prefill_chunked(const void* q, const void* k, const void* v, int qkv_dtype, const void* ga,
                                   const void* gb, int gb_dtype, int64_t gate_stride, const float* A_log,
                                   const float* dt_bias, int gate_mode, const float* state_in,
                                   float* state_out, void* y, int y_dtype,
                                   const int32_t* cu_seqlens, int N, int64_t T_total, int Hk,
                                   int Hv, int Dk, int Dv, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
    GDN_REQUIRE(N > 0 && T_total >= 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0,
                "gdn_prefill_chunked: bad sizes");
    if (Dk != kHD || Dv != kHD)
        return fail(GDN_EUNSUPPORTED, "gdn_prefill_chunked: specialised for Dk=Dv=128 (got %d, %d)", Dk, Dv);
    GDN_REQUIRE(gate_mode == 0 || gate_mode == 1, "gdn_prefill_chunked: gate_mode must be 0 or 1");
    GDN_REQUIRE(gate_stride >= Hv, "gdn_prefill_chunked: gate_stride %lld below Hv=%d",
                (long long)gate_stride, Hv);
    GDN_REQUIRE(valid_dtype(gb_dtype) && valid_dtype(y_dtype), "gdn_prefill_chunked: bad dtype");
    if (qkv_dtype != GDN_BF16 && qkv_dtype != GDN_F32)
        return fail(GDN_EUNSUPPORTED, "gdn_prefill_chunked: q, k, v must be bfloat16 or float32");
    const bool f32 = qkv_dtype == GDN_F32;
    GDN_REQUIRE(gate_mode == 1 || (A_log && dt_bias), "gdn_prefill_chunked: gate_mode 0 needs A_log, dt_bias");
    GDN_REQUIRE(cu_seqlens || T_total % N == 0, "gdn_prefill_chunked: T_total not divisible by N");
    GDN_REQUIRE(T_total < (int64_t(1) << 31), "gdn_prefill_chunked: token count must fit int32");
    GDN_REQUIRE(state_out, "gdn_prefill_chunked: null state_out");
    GDN_REQUIRE(T_total == 0 || (q && k && v && ga && gb && y), "gdn_prefill_chunked: null pointer");
    GDN_REQUIRE((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                 reinterpret_cast<uintptr_t>(state_in) | reinterpret_cast<uintptr_t>(state_out) |
                 reinterpret_cast<uintptr_t>(workspace)) % 16 == 0,
                "gdn_prefill_chunked: q, k, states and workspace must be 16-byte aligned");
    GDN_REQUIRE(reinterpret_cast<uintptr_t>(v) % (f32 ? 16 : 8) == 0,
                "gdn_prefill_chunked: v must be %d-byte aligned", f32 ? 16 : 8);
    const int64_t need = records_offset(N) + chunks_bound(T_total, N) * Hv * kRecBytes;
    GDN_REQUIRE(workspace && workspace_bytes >= need,
                "gdn_prefill_chunked: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)need);
    if (state_in && state_in != state_out) {
        const int64_t sb = int64_t(N) * Hv * kHD * kHD * 4;
        GDN_REQUIRE(!overlaps(state_in, sb, state_out, sb), "gdn_prefill_chunked: states overlap");
    }
    GDN_REQUIRE(state_in != state_out, "gdn_prefill_chunked: state_out must not alias state_in");

    hipStream_t s = as_stream(stream);
    RunLayout rl;
    rl.cu = cu_seqlens;
    rl.N = N;
    rl.L_uniform = cu_seqlens ? 0 : T_total / N;
    rl.cpr = int((rl.L_uniform + kChunk - 1) / kChunk);
    rl.chunk_off = nullptr;
    char* records = static_cast<char*>(workspace) + records_offset(N);
    if (cu_seqlens) {  // packed runs: chunk offsets from the run lengths
        int32_t* chunk_off = static_cast<int32_t*>(workspace);
        hipLaunchKernelGGL(chunk_offsets_kernel, dim3(1), dim3(64), 0, s, cu_seqlens, N, chunk_off);
        if (int rc = check_launch("gdn_prefill_chunked/offsets")) return rc;
        rl.chunk_off = chunk_off;
    }
    const int64_t nchunks = chunks_bound(T_total, N);
    const int64_t items = (nchunks * Hk + 7) / 8 * 8;
    // value heads per chunk workgroup: with float32 input two where a key
    // head has an even number (with bf16 input the second head's products
    // would spill)
    const bool pairs = f32 && (Hv / Hk) % 2 == 0;
    const dim3 cgrid(unsigned(items * (Hv / Hk) / (pairs ? 2 : 1)));
    hipLaunchKernelGGL(f32 ? (pairs ? prefill_chunk_f32_kernel<2> : prefill_chunk_f32_kernel<1>) : prefill_chunk_kernel,
                       cgrid, dim3(256), 0, s, q, k, ga, gb,
                       gb_dtype, gate_stride, A_log, dt_bias, gate_mode, rl, records, Hk, Hv);
    if (int rc = check_launch("gdn_prefill_chunked/chunk")) return rc;
    const dim3 sgrid(unsigned(int64_t(N) * Hv * kSlices));
#define GDN_STATE_LAUNCH(YT, F32)                                                                 \
    hipLaunchKernelGGL((prefill_state_kernel<YT, F32>), sgrid, dim3(kStateThreads), 0, s, q, k, v, \
                       state_in, state_out, static_cast<YT::storage*>(y), rl, records, Hk, Hv)
    if (f32) {
        if (y_dtype == GDN_F32) GDN_STATE_LAUNCH(ActF32, true);
        else if (y_dtype == GDN_BF16) GDN_STATE_LAUNCH(ActBF16, true);
        else GDN_STATE_LAUNCH(ActF16, true);
    } else {
        if (y_dtype == GDN_F32) GDN_STATE_LAUNCH(ActF32, false);
        else if (y_dtype == GDN_BF16) GDN_STATE_LAUNCH(ActBF16, false);
        else GDN_STATE_LAUNCH(ActF16, false);
    }
#undef GDN_STATE_LAUNCH
    return check_launch("gdn_prefill_chunked/state");
}

namespace {

// The fused prefill's q, k and v (bf16) follow the chunked prefill's workspace.
int64_t fused_qkv_offset(int N, int64_t T_total, int Hv) {
    return (records_offset(N) + chunks_bound(T_total, N) * Hv * kRecBytes + 255) & ~int64_t(255);
}

}  // namespace

extern "C" int64_t gdn_prefill_fused_workspace_size(int N, int64_t T_total, int Hk, int Hv, int Dk, int Dv) {
    if (N <= 0 || T_total < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk)
        return fail(GDN_EINVAL, "gdn_prefill_fused_workspace_size: bad sizes");
    if (Dk != kHD || Dv != kHD)
        return fail(GDN_EUNSUPPORTED, "gdn_prefill_fused_workspace_size: specialised for Dk=Dv=128");
    return fused_qkv_offset(N, T_total, Hv) + T_total * (2LL * Hk + Hv) * kHD * 2;
}

extern "C" int gdn_prefill_fused(const void* qkv, int64_t qkv_stride, const void* conv_state_in,
                                 void* conv_state_out, int conv_dtype, const float* conv_weight, int K,
                                 const void* a, const void* b, int gate_dtype, int64_t gate_stride,
                                 const float* A_log, const float* dt_bias, const float* state_in,
                                 float* state_out, void* y, int y_dtype, const int32_t* cu_seqlens, int N,
                                 int64_t T_total, int Hk, int Hv, int Dk, int Dv, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
    GDN_REQUIRE(N > 0 && T_total >= 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0, "gdn_prefill_fused: bad sizes");
    if (Dk != kHD || Dv != kHD || K != 4)
        return fail(GDN_EUNSUPPORTED, "gdn_prefill_fused: specialised for Dk=Dv=128, K=4 (got %d, %d, %d)",
                    Dk, Dv, K);
    if (conv_dtype != GDN_BF16 && conv_dtype != GDN_F32)
        return fail(GDN_EUNSUPPORTED, "gdn_prefill_fused: conv state must be bfloat16 or float32");
    GDN_REQUIRE(valid_dtype(gate_dtype) && valid_dtype(y_dtype), "gdn_prefill_fused: bad dtype");
    GDN_REQUIRE(gate_stride >= Hv, "gdn_prefill_fused: gate_stride %lld below Hv=%d", (long long)gate_stride,
                Hv);
    GDN_REQUIRE(cu_seqlens || T_total % N == 0, "gdn_prefill_fused: T_total not divisible by N");
    GDN_REQUIRE(T_total < (int64_t(1) << 31), "gdn_prefill_fused: token count must fit int32");
    const int64_t C = (2LL * Hk + Hv) * kHD;
    GDN_REQUIRE(qkv_stride >= C && qkv_stride % 8 == 0,
                "gdn_prefill_fused: qkv_stride %lld must be at least conv_dim %lld and a multiple of 8",
                (long long)qkv_stride, (long long)C);
    GDN_REQUIRE(state_out && conv_state_in && conv_state_out && conv_weight && A_log && dt_bias,
                "gdn_prefill_fused: null pointer");
    GDN_REQUIRE(T_total == 0 || (qkv && a && b && y), "gdn_prefill_fused: null pointer");
    const auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    GDN_REQUIRE(al(qkv) && al(conv_state_in) && al(conv_state_out) && al(conv_weight) && al(state_in) &&
                    al(state_out) && al(workspace),
                "gdn_prefill_fused: qkv, conv states, conv weight, states and workspace must be 16-byte aligned");
    const int64_t qkv_off = fused_qkv_offset(N, T_total, Hv);
    const int64_t need = qkv_off + T_total * C * 2;
    GDN_REQUIRE(workspace && workspace_bytes >= need, "gdn_prefill_fused: workspace of %lld bytes, need %lld",
                (long long)workspace_bytes, (long long)need);
    const int64_t cb = int64_t(N) * 3 * C;
    GDN_REQUIRE(!overlaps(conv_state_in, cb * dtype_size(conv_dtype), conv_state_out, cb * 2),
                "gdn_prefill_fused: conv_state_out overlaps conv_state_in");
    GDN_REQUIRE(state_in != state_out, "gdn_prefill_fused: state_out must not alias state_in");
    if (state_in) {
        const int64_t sb = int64_t(N) * Hv * kHD * kHD * 4;
        GDN_REQUIRE(!overlaps(state_in, sb, state_out, sb), "gdn_prefill_fused: states overlap");
    }

    hipStream_t s = as_stream(stream);
    RunLayout rl;
    rl.cu = cu_seqlens;
    rl.N = N;
    rl.L_uniform = cu_seqlens ? 0 : T_total / N;
    rl.cpr = int((rl.L_uniform + kChunk - 1) / kChunk);
    rl.chunk_off = nullptr;
    char* ws = static_cast<char*>(workspace);
    char* records = ws + records_offset(N);
    if (cu_seqlens) {
        int32_t* chunk_off = reinterpret_cast<int32_t*>(ws);
        hipLaunchKernelGGL(chunk_offsets_kernel, dim3(1), dim3(64), 0, s, cu_seqlens, N, chunk_off);
        if (int rc = check_launch("gdn_prefill_fused/offsets")) return rc;
        rl.chunk_off = chunk_off;
    }
    ConvIn cv;
    cv.qkv = static_cast<const uint16_t*>(qkv);
    cv.qs = qkv_stride;
    cv.cs_in = conv_state_in;
    cv.cs_out = static_cast<uint16_t*>(conv_state_out);
    cv.w = conv_weight;
    cv.qo = reinterpret_cast<uint16_t*>(ws + qkv_off);
    cv.ko = cv.qo + T_total * Hk * kHD;
    cv.vo = cv.ko + T_total * Hk * kHD;
    const int64_t items = (chunks_bound(T_total, N) * Hk + 7) / 8 * 8;
    const dim3 cgrid(unsigned(items * (Hv / Hk)));
    if (conv_dtype == GDN_F32)
        hipLaunchKernelGGL(prefill_chunk_conv_kernel<GDN_F32>, cgrid, dim3(256), 0, s, a, b, gate_dtype,
                           gate_stride, A_log, dt_bias, rl, records, Hk, Hv, cv);
    else
        hipLaunchKernelGGL(prefill_chunk_conv_kernel<GDN_BF16>, cgrid, dim3(256), 0, s, a, b, gate_dtype,
                           gate_stride, A_log, dt_bias, rl, records, Hk, Hv, cv);
    if (int rc = check_launch("gdn_prefill_fused/chunk")) return rc;
    if (cu_seqlens || T_total == 0) {  // runs without tokens keep their conv state
        if (conv_dtype == GDN_F32)
            hipLaunchKernelGGL(conv_state_empty_runs_kernel<GDN_F32>, dim3(unsigned(N)), dim3(256), 0, s, rl, cv,
                               int(C));
        else
            hipLaunchKernelGGL(conv_state_empty_runs_kernel<GDN_BF16>, dim3(unsigned(N)), dim3(256), 0, s, rl,
                               cv, int(C));
        if (int rc = check_launch("gdn_prefill_fused/conv_state")) return rc;
    }
    const dim3 sgrid(unsigned(int64_t(N) * Hv * kSlices));
#define GDN_STATE_LAUNCH(YT)                                                                            \
    hipLaunchKernelGGL((prefill_state_kernel<YT, false>), sgrid, dim3(kStateThreads), 0, s, cv.qo, cv.ko, \
                       cv.vo, state_in, state_out, static_cast<YT::storage*>(y), rl, records, Hk, Hv)
    if (y_dtype == GDN_F32) GDN_STATE_LAUNCH(ActF32);
    else if (y_dtype == GDN_BF16) GDN_STATE_LAUNCH(ActBF16);
    else GDN_STATE_LAUNCH(ActF16);
#undef GDN_STATE_LAUNCH
    return check_launch("gdn_prefill_fused/state");
}
