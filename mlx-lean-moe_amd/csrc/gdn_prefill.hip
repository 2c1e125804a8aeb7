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
//     records Tb and P = lower(Q K^T o G) (each bf16 hi + lo) plus l.
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
#include "gdn_host.h"

namespace gdn {

constexpr int kChunk = 64;
constexpr int kHD = 128;                 // Dk = Dv
constexpr int kSliceRows = 16;           // state rows per state-pass workgroup
constexpr int kSlices = kHD / kSliceRows;
constexpr int kMaxGroup = 8;             // value heads per key head handled by the chunk pass
constexpr float kLogGateFloor = -80.f;   // exp(-80) ~ 1.8e-35: a reset state

// Per (chunk, value head) record written by the chunk pass.
constexpr int64_t kMatBytes = int64_t(kChunk) * kChunk * 2;
constexpr int64_t kRecTbHi = 0, kRecTbLo = kMatBytes, kRecPHi = 2 * kMatBytes, kRecPLo = 3 * kMatBytes;
constexpr int64_t kRecL = 4 * kMatBytes;
constexpr int64_t kRecBytes = 4 * kMatBytes + kChunk * 4;

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

GDN_DEV bf16x8 load8(const uint16_t* p) { return *reinterpret_cast<const bf16x8*>(p); }

GDN_DEV bf16x8 zero8() {
    bf16x8 z;
#pragma unroll
    for (int j = 0; j < 8; ++j) z[j] = __bf16(0.f);
    return z;
}

// ---------------------------------------------------------------------------
// run / chunk bookkeeping
// ---------------------------------------------------------------------------

// chunk_off[i] = index of run i's first chunk; chunk_off[N] = chunk count.
__global__ void chunk_offsets_kernel(const int32_t* __restrict__ cu, int N, int64_t L_uniform,
                                     int32_t* __restrict__ chunk_off) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    int32_t off = 0;
    for (int i = 0; i < N; ++i) {
        chunk_off[i] = off;
        const int64_t len = cu ? int64_t(cu[i + 1]) - cu[i] : L_uniform;
        off += int32_t((len + kChunk - 1) / kChunk);
    }
    chunk_off[N] = off;
}

struct ChunkPos {
    int run;
    int64_t t0;  // first token
    int len;     // tokens in the chunk (1..64)
};

GDN_DEV ChunkPos locate_chunk(const int32_t* chunk_off, const int32_t* cu, int N, int64_t L_uniform,
                              int g) {
    const int run = find_run(chunk_off, N, g);
    const int c = g - chunk_off[run];
    const int64_t rs = cu ? cu[run] : run * L_uniform;
    const int64_t re = cu ? cu[run + 1] : rs + L_uniform;
    const int64_t t0 = rs + int64_t(c) * kChunk;
    const int64_t len = re - t0 < kChunk ? re - t0 : kChunk;
    return {run, t0, int(len)};
}

// ---------------------------------------------------------------------------
// chunk pass
// ---------------------------------------------------------------------------

constexpr int kKS = kHD + 8;    // bf16 row stride of the K/Q tiles
constexpr int kFS = kChunk + 1; // float row stride of the A/T tiles

// One wave: acc += A_blk * B_blk for 16 x 16 blocks held in LDS with row
// stride kFS; lane (m = l/4, n0 = 4 (l%4)) owns acc = out[m][n0..n0+3].
GDN_DEV void block_mma(float (&acc)[4], const float* A, const float* B, int m, int n0) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float a = A[m * kFS + k];
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] += a * B[k * kFS + n0 + q];
    }
}

__global__ __launch_bounds__(256) void prefill_chunk_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const void* __restrict__ ga,
    const void* __restrict__ gb, int gb_dtype, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, int gate_mode, const int32_t* __restrict__ cu, int N,
    int64_t L_uniform, const int32_t* __restrict__ chunk_off, char* __restrict__ records, int Hk,
    int Hv) {
    // K/Q tiles first; once K K^T and Q K^T are in registers the same bytes
    // hold the A and T matrices of one value head at a time.
    __shared__ __attribute__((aligned(16))) char smem[2 * kChunk * kKS * 2];
    __shared__ float l_sh[kMaxGroup][kChunk], beta_sh[kMaxGroup][kChunk];
    __shared__ float wtmp[4][16 * kFS];
    uint16_t* Ks = reinterpret_cast<uint16_t*>(smem);
    uint16_t* Qs = Ks + kChunk * kKS;
    float* As = reinterpret_cast<float*>(smem);
    float* Ts = As + kChunk * kFS;

    const int g = blockIdx.x, hk = blockIdx.y;
    if (g >= chunk_off[N]) return;
    const ChunkPos pos = locate_chunk(chunk_off, cu, N, L_uniform, g);
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int r = Hv / Hk;

    // K and Q of the chunk (rows past the run are zero).
    for (int idx = tid; idx < kChunk * (kHD / 8); idx += 256) {
        const int row = idx / (kHD / 8), seg = idx % (kHD / 8);
        uint4 kv = {0, 0, 0, 0}, qv = {0, 0, 0, 0};
        if (row < pos.len) {
            const int64_t off = ((pos.t0 + row) * Hk + hk) * kHD + seg * 8;
            kv = *reinterpret_cast<const uint4*>(k + off);
            qv = *reinterpret_cast<const uint4*>(q + off);
        }
        *reinterpret_cast<uint4*>(Ks + row * kKS + seg * 8) = kv;
        *reinterpret_cast<uint4*>(Qs + row * kKS + seg * 8) = qv;
    }
    // Gates of the group's value heads: lane = token; l = inclusive prefix sum of log g.
    for (int e = w; e < r; e += 4) {
        const int hv = hk * r + e;
        float lg = 0.f, beta = 0.f;
        if (l < pos.len) {
            const int64_t i = (pos.t0 + l) * Hv + hv;
            if (gate_mode == 0) {
                lg = log_forget_gate(load_any(ga, i, gb_dtype), A_log[hv], dt_bias[hv]);
                beta = round_to(sigmoid(load_any(gb, i, gb_dtype)), gb_dtype);
            } else {
                const float gv = static_cast<const float*>(ga)[i];
                lg = gv > 0.f ? logf(gv) : kLogGateFloor;
                beta = load_any(gb, i, gb_dtype);
            }
            lg = fmaxf(lg, kLogGateFloor);
        }
#pragma unroll
        for (int off = 1; off < kChunk; off <<= 1) {
            const float y = __shfl_up(lg, off, kWave);
            if (l >= off) lg += y;
        }
        l_sh[e][l] = lg;
        beta_sh[e][l] = beta;
        reinterpret_cast<float*>(records + (int64_t(g) * Hv + hv) * kRecBytes + kRecL)[l] = lg;
    }
    __syncthreads();

    // K K^T and Q K^T: wave w owns token rows 16w..16w+15, all four column tiles.
    f32x4 kk[4], qk[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) kk[jt] = qk[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int lr = l & 15, lg8 = 8 * (l >> 4);
#pragma unroll
    for (int s = 0; s < kHD / 32; ++s) {
        const bf16x8 ak = load8(Ks + (16 * w + lr) * kKS + 32 * s + lg8);
        const bf16x8 aq = load8(Qs + (16 * w + lr) * kKS + 32 * s + lg8);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            const bf16x8 bk = load8(Ks + (16 * jt + lr) * kKS + 32 * s + lg8);
            kk[jt] = mfma16(ak, bk, kk[jt]);
            qk[jt] = mfma16(aq, bk, qk[jt]);
        }
    }
    __syncthreads();  // K/Q tiles are dead from here on

    const int m = l >> 2, n0 = 4 * (l & 3);
    for (int e = 0; e < r; ++e) {
        const int hv = hk * r + e;
        char* rec = records + (int64_t(g) * Hv + hv) * kRecBytes;
        uint16_t* rec_ph = reinterpret_cast<uint16_t*>(rec + kRecPHi);
        uint16_t* rec_pl = reinterpret_cast<uint16_t*>(rec + kRecPLo);
        // P and A from the accumulators: element (i, j) with
        // i = 16w + 4(l/16) + ii, j = 16jt + l%16.
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int i = 16 * w + 4 * (l >> 4) + ii, j = 16 * jt + lr;
                const float dec = i >= j ? expf(l_sh[e][i] - l_sh[e][j]) : 0.f;
                split_bf16(qk[jt][ii] * dec, rec_ph[i * kChunk + j], rec_pl[i * kChunk + j]);
                As[i * kFS + j] = i > j ? beta_sh[e][i] * kk[jt][ii] * dec : 0.f;
            }
        }
        __syncthreads();

        // T = (I + A)^-1 by 16 x 16 blocks. Diagonal blocks by forward
        // substitution (lane n < 16 owns column n).
        if (l < 16) {
            float col[16];
#pragma unroll
            for (int mm = 0; mm < 16; ++mm) col[mm] = mm == l ? 1.f : 0.f;
            const float* Ab = As + (16 * w) * kFS + 16 * w;
#pragma unroll
            for (int mm = 1; mm < 16; ++mm) {
                float sum = 0.f;
#pragma unroll
                for (int kk2 = 0; kk2 < mm; ++kk2) sum += Ab[mm * kFS + kk2] * col[kk2];
                if (mm > l) col[mm] = -sum;
            }
            float* Tb = Ts + (16 * w) * kFS + 16 * w;
#pragma unroll
            for (int mm = 0; mm < 16; ++mm) Tb[mm * kFS + l] = col[mm];
        }
        __syncthreads();
        // Off-diagonal blocks by block diagonals: T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj.
        for (int dist = 1; dist < 4; ++dist) {
            const int bj = w, bi = w + dist;
            const bool active = bi < 4;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            if (active) {
                for (int bk = bj; bk < bi; ++bk)
                    block_mma(acc, As + (16 * bi) * kFS + 16 * bk, Ts + (16 * bk) * kFS + 16 * bj, m, n0);
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) wtmp[w][m * kFS + n0 + qq] = acc[qq];
            }
            __syncthreads();
            if (active) {
                float out[4] = {0.f, 0.f, 0.f, 0.f};
                block_mma(out, Ts + (16 * bi) * kFS + 16 * bi, wtmp[w], m, n0);
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) Ts[(16 * bi + m) * kFS + 16 * bj + n0 + qq] = -out[qq];
            }
            __syncthreads();
        }
        // Tb = T diag(beta), split into bf16 hi + lo.
        uint16_t* tb_hi = reinterpret_cast<uint16_t*>(rec + kRecTbHi);
        uint16_t* tb_lo = reinterpret_cast<uint16_t*>(rec + kRecTbLo);
        for (int idx = tid; idx < kChunk * kChunk; idx += 256) {
            const int i = idx / kChunk, j = idx % kChunk;
            const float t = i == j ? 1.f : (i > j ? Ts[i * kFS + j] : 0.f);
            uint16_t hi, lo;
            split_bf16(t * beta_sh[e][j], hi, lo);
            tb_hi[idx] = hi;
            tb_lo[idx] = lo;
        }
        __syncthreads();  // As / Ts are reused by the next value head
    }
}

// ---------------------------------------------------------------------------
// state pass
// ---------------------------------------------------------------------------

constexpr int kSS = kHD + 8;     // bf16 row stride of the S^T operand tiles
constexpr int kTS = kChunk + 8;  // bf16 row stride of token-major operand tiles

// One chunk's operands as this lane needs them (fetched a chunk ahead).
struct ChunkOperands {
    bf16x8 ka[4], qa[4];    // K / Q rows 16w + l%16, dk 32s + 8(l/16) .. +7
    bf16x8 tbh[2], tbl[2];  // Tb rows 16w + l%16 (hi, lo), tokens 32s + 8(l/16) .. +7
    bf16x8 pah[2], pal[2];  // P rows 16w + l%16 (hi, lo)
    uint32_t v[4];          // V (bf16 bits) at (token 16w + 4(l/16) + i, dv0 + l%16)
    float l;                // l[tid] (tid < 64)
};

struct StatePassCtx {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const char* records;
    int64_t rs, re, qk_stride;
    int c0, h, hk, Hv, dv0;
};

// Every load is unconditional, from a token index clamped into the chunk: a
// divergent conditional load would make the compiler wait for all
// outstanding loads (the prefetch included), and consuming a loaded value
// here would do the same. Rows past the run then hold copies of the last
// token, which contribute nothing: their beta and log-decay are zero, so
// their columns of Tb and P and their rows of D vanish.
GDN_DEV void fetch_chunk(ChunkOperands& op, const StatePassCtx& cx, int c, int tid, int w, int lr,
                         int lq, int lg8) {
    const int64_t t0 = cx.rs + int64_t(c) * kChunk;
    const int len = cx.re - t0 < kChunk ? int(cx.re - t0) : kChunk;
    const char* rec = cx.records + (int64_t(cx.c0 + c) * cx.Hv + cx.h) * kRecBytes;
    const int tok = 16 * w + lr;
    const int tok_c = tok < len ? tok : len - 1;
    const int64_t base = (t0 + tok_c) * cx.qk_stride + cx.hk * kHD + lg8;
#pragma unroll
    for (int s = 0; s < kHD / 32; ++s) {
        op.ka[s] = load8(cx.k + base + 32 * s);
        op.qa[s] = load8(cx.q + base + 32 * s);
    }
    const uint16_t* tb_hi = reinterpret_cast<const uint16_t*>(rec + kRecTbHi);
    const uint16_t* tb_lo = reinterpret_cast<const uint16_t*>(rec + kRecTbLo);
    const uint16_t* p_hi = reinterpret_cast<const uint16_t*>(rec + kRecPHi);
    const uint16_t* p_lo = reinterpret_cast<const uint16_t*>(rec + kRecPLo);
#pragma unroll
    for (int s = 0; s < kChunk / 32; ++s) {
        op.tbh[s] = load8(tb_hi + tok * kChunk + 32 * s + lg8);
        op.tbl[s] = load8(tb_lo + tok * kChunk + 32 * s + lg8);
        op.pah[s] = load8(p_hi + tok * kChunk + 32 * s + lg8);
        op.pal[s] = load8(p_lo + tok * kChunk + 32 * s + lg8);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tv = 16 * w + 4 * lq + i;
        const int tv_c = tv < len ? tv : len - 1;
        op.v[i] = cx.v[((t0 + tv_c) * cx.Hv + cx.h) * kHD + cx.dv0 + lr];
    }
    op.l = reinterpret_cast<const float*>(rec + kRecL)[tid & (kChunk - 1)];
}

GDN_DEV uint2 pack4(const uint16_t (&x)[4]) {
    return uint2{uint32_t(x[0]) | (uint32_t(x[1]) << 16), uint32_t(x[2]) | (uint32_t(x[3]) << 16)};
}

struct StatePassLds {
    uint16_t Ss_hi[kSliceRows * kSS], Ss_lo[kSliceRows * kSS];
    uint16_t Kt[kHD * kTS];
    uint16_t Rs_hi[kSliceRows * kTS], Rs_lo[kSliceRows * kTS];
    uint16_t Ds_hi[kSliceRows * kTS], Ds_lo[kSliceRows * kTS];
    uint16_t D2_hi[kSliceRows * kTS], D2_lo[kSliceRows * kTS];
    float l[kChunk];
};

// Chunk step, part 1: the S^T operand (hi + lo), the chunk's K^T and its
// log-decays into LDS. Consuming the chunk's K registers and l here means its
// loads are complete before the next chunk's prefetch is issued.
GDN_DEV void stage_chunk(const ChunkOperands& op, const f32x4 (&acc)[2], StatePassLds& sm, int tid,
                         int w, int lr, int lq, int lg8) {
    __syncthreads();  // the previous chunk's readers of the LDS tiles are done
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int dk = 32 * w + 16 * t + 4 * lq;
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) split_bf16(acc[t][i], hi[i], lo[i]);
        *reinterpret_cast<uint2*>(sm.Ss_hi + lr * kSS + dk) = pack4(hi);
        *reinterpret_cast<uint2*>(sm.Ss_lo + lr * kSS + dk) = pack4(lo);
    }
    {
        const int tok = 16 * w + lr;
#pragma unroll
        for (int s = 0; s < kHD / 32; ++s) {
            // Whole-vector bit cast: this compiler miscompiles a bit cast of a
            // single __bf16 vector element (it repeats element 0).
            const u16x8 kv = __builtin_bit_cast(u16x8, op.ka[s]);
#pragma unroll
            for (int j = 0; j < 8; ++j) sm.Kt[(32 * s + lg8 + j) * kTS + tok] = kv[j];
        }
    }
    sm.l[tid & (kChunk - 1)] = op.l;  // all four waves store the same values: no branch
    __syncthreads();
}

// Chunk step, part 2: S^T (acc) advances by the chunk, y is written.
template <class Y>
GDN_DEV void compute_chunk(const ChunkOperands& op, f32x4 (&acc)[2], StatePassLds& sm,
                           const StatePassCtx& cx, int c, typename Y::storage* __restrict__ y,
                           int w, int lr, int lq, int lg8) {
    const int64_t t0 = cx.rs + int64_t(c) * kChunk;
    const int len = cx.re - t0 < kChunk ? int(cx.re - t0) : kChunk;

    // X_K = K S^T, X_Q = Q S^T (S in hi + lo): token rows 16w..16w+15, the
    // hi and lo products in separate accumulators (shorter dependency chains).
    f32x4 xk = {0.f, 0.f, 0.f, 0.f}, xk2 = xk, xq = xk, xq2 = xk;
#pragma unroll
    for (int s = 0; s < kHD / 32; ++s) {
        const bf16x8 bh = load8(sm.Ss_hi + lr * kSS + 32 * s + lg8);
        const bf16x8 bl = load8(sm.Ss_lo + lr * kSS + 32 * s + lg8);
        xk = mfma16(op.ka[s], bh, xk);
        xk2 = mfma16(op.ka[s], bl, xk2);
        xq = mfma16(op.qa[s], bh, xq);
        xq2 = mfma16(op.qa[s], bl, xq2);
    }
    xk += xk2;
    xq += xq2;
    // R = V - exp(l) X_K, stored hi + lo as R[dv][token].
    float el[4];
    {
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            el[i] = expf(sm.l[16 * w + 4 * lq + i]);
            split_bf16(bf16_bits_to_f32(op.v[i]) - el[i] * xk[i], hi[i], lo[i]);
        }
        const int tok0 = 16 * w + 4 * lq;
        *reinterpret_cast<uint2*>(sm.Rs_hi + lr * kTS + tok0) = pack4(hi);
        *reinterpret_cast<uint2*>(sm.Rs_lo + lr * kTS + tok0) = pack4(lo);
    }
    __syncthreads();

    // D = Tb R, three products (hi.hi + hi.lo + lo.hi) in two accumulators.
    f32x4 d = {0.f, 0.f, 0.f, 0.f}, d2 = d;
#pragma unroll
    for (int s = 0; s < kChunk / 32; ++s) {
        const bf16x8 bh = load8(sm.Rs_hi + lr * kTS + 32 * s + lg8);
        const bf16x8 bl = load8(sm.Rs_lo + lr * kTS + 32 * s + lg8);
        d = mfma16(op.tbh[s], bh, d);
        d2 = mfma16(op.tbh[s], bl, d2);
        d2 = mfma16(op.tbl[s], bh, d2);
    }
    d += d2;
    // D (hi + lo, for Y) and D'' = exp(l_C - l) D (hi + lo, for the update).
    const float lC = sm.l[kChunk - 1];
    {
        uint16_t dh[4], dl[4], hi[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            split_bf16(d[i], dh[i], dl[i]);
            split_bf16(expf(lC - sm.l[16 * w + 4 * lq + i]) * d[i], hi[i], lo[i]);
        }
        const int tok0 = 16 * w + 4 * lq;
        *reinterpret_cast<uint2*>(sm.Ds_hi + lr * kTS + tok0) = pack4(dh);
        *reinterpret_cast<uint2*>(sm.Ds_lo + lr * kTS + tok0) = pack4(dl);
        *reinterpret_cast<uint2*>(sm.D2_hi + lr * kTS + tok0) = pack4(hi);
        *reinterpret_cast<uint2*>(sm.D2_lo + lr * kTS + tok0) = pack4(lo);
    }
    __syncthreads();

    // Y = exp(l) X_Q + P D.
    {
        f32x4 yacc;
#pragma unroll
        for (int i = 0; i < 4; ++i) yacc[i] = el[i] * xq[i];
        f32x4 y2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kChunk / 32; ++s) {
            const bf16x8 bh = load8(sm.Ds_hi + lr * kTS + 32 * s + lg8);
            const bf16x8 bl = load8(sm.Ds_lo + lr * kTS + 32 * s + lg8);
            yacc = mfma16(op.pah[s], bh, yacc);
            y2 = mfma16(op.pah[s], bl, y2);
            y2 = mfma16(op.pal[s], bh, y2);
        }
        yacc += y2;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = 16 * w + 4 * lq + i;
            if (tok < len) Y::store(y, ((t0 + tok) * cx.Hv + cx.h) * kHD + cx.dv0 + lr, yacc[i]);
        }
    }
    // S^T <- exp(l_C) S^T + K^T D'' (D'' in hi + lo).
    const float eC = expf(lC);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        acc[t] *= eC;
        f32x4 lo_acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kChunk / 32; ++s) {
            const bf16x8 a = load8(sm.Kt + (32 * w + 16 * t + lr) * kTS + 32 * s + lg8);
            acc[t] = mfma16(a, load8(sm.D2_hi + lr * kTS + 32 * s + lg8), acc[t]);
            lo_acc = mfma16(a, load8(sm.D2_lo + lr * kTS + 32 * s + lg8), lo_acc);
        }
        acc[t] += lo_acc;
    }
}

template <class Y>
__global__ __launch_bounds__(256) void prefill_state_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ state_in, float* __restrict__ state_out,
    typename Y::storage* __restrict__ y, const int32_t* __restrict__ cu, int N, int64_t L_uniform,
    const int32_t* __restrict__ chunk_off, const char* __restrict__ records, int Hk, int Hv) {
    __shared__ __attribute__((aligned(16))) StatePassLds sm;

    // Work mapping: the 8 slices of one (run, head) share its K/Q and chunk
    // records, so they are placed on one XCD (workgroups go round-robin over
    // the 8 XCDs) when the head count allows it.
    const int R = N * Hv;
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
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int lr = l & 15, lq = l >> 4, lg8 = 8 * lq;

    StatePassCtx cx;
    cx.q = q;
    cx.k = k;
    cx.v = v;
    cx.records = records;
    cx.rs = cu ? cu[run] : run * L_uniform;
    cx.re = cu ? cu[run + 1] : cx.rs + L_uniform;
    cx.qk_stride = int64_t(Hk) * kHD;
    cx.c0 = chunk_off[run];
    cx.h = h;
    cx.hk = h / (Hv / Hk);
    cx.Hv = Hv;
    cx.dv0 = slice * kSliceRows;
    const int nch = chunk_off[run + 1] - cx.c0;

    // S^T tile in accumulators: acc[t][i] = S^T[dk = 32w + 16t + 4(l/16) + i][dv = dv0 + l%16].
    f32x4 acc[2];
    const int64_t sbase = ((int64_t(run) * Hv + h) * kHD + cx.dv0 + lr) * kHD;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int dk = 32 * w + 16 * t + 4 * lq;
        if (state_in) {
            const float4 s4 = *reinterpret_cast<const float4*>(state_in + sbase + dk);
            acc[t] = f32x4{s4.x, s4.y, s4.z, s4.w};
        } else {
            acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }

    // Two operand sets, alternated: chunk c computes from one while chunk
    // c + 1's loads land in the other.
    ChunkOperands opa, opb;
    if (nch > 0) fetch_chunk(opa, cx, 0, tid, w, lr, lq, lg8);
    for (int c = 0; c < nch; c += 2) {
        stage_chunk(opa, acc, sm, tid, w, lr, lq, lg8);
        if (c + 1 < nch) fetch_chunk(opb, cx, c + 1, tid, w, lr, lq, lg8);
        compute_chunk<Y>(opa, acc, sm, cx, c, y, w, lr, lq, lg8);
        if (c + 1 >= nch) break;
        stage_chunk(opb, acc, sm, tid, w, lr, lq, lg8);
        if (c + 2 < nch) fetch_chunk(opa, cx, c + 2, tid, w, lr, lq, lg8);
        compute_chunk<Y>(opb, acc, sm, cx, c + 1, y, w, lr, lq, lg8);
    }

#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int dk = 32 * w + 16 * t + 4 * lq;
        *reinterpret_cast<float4*>(state_out + sbase + dk) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
    }
}

}  // namespace gdn

using namespace gdn;

extern "C" int64_t gdn_prefill_workspace_size(int N, int64_t T_total, int Hk, int Hv, int Dk, int Dv) {
    if (N <= 0 || T_total < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return fail(GDN_EINVAL, "gdn_prefill_workspace_size: bad sizes");
    if (Dk != kHD || Dv != kHD) return fail(GDN_EUNSUPPORTED, "gdn_prefill_workspace_size: specialised for Dk=Dv=128");
    return records_offset(N) + chunks_bound(T_total, N) * Hv * kRecBytes;
}

extern "C" int gdn_prefill_chunked(const void* q, const void* k, const void* v, const void* ga,
                                   const void* gb, int gb_dtype, const float* A_log,
                                   const float* dt_bias, int gate_mode, const float* state_in,
                                   float* state_out, void* y, int y_dtype,
                                   const int32_t* cu_seqlens, int N, int64_t T_total, int Hk,
                                   int Hv, int Dk, int Dv, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
    GDN_REQUIRE(N > 0 && T_total >= 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0,
                "gdn_prefill_chunked: bad sizes");
    if (Dk != kHD || Dv != kHD)
        return fail(GDN_EUNSUPPORTED, "gdn_prefill_chunked: specialised for Dk=Dv=128 (got %d, %d)", Dk, Dv);
    GDN_REQUIRE(Hv / Hk <= kMaxGroup, "gdn_prefill_chunked: more than %d value heads per key head", kMaxGroup);
    GDN_REQUIRE(gate_mode == 0 || gate_mode == 1, "gdn_prefill_chunked: gate_mode must be 0 or 1");
    GDN_REQUIRE(valid_dtype(gb_dtype) && valid_dtype(y_dtype), "gdn_prefill_chunked: bad dtype");
    GDN_REQUIRE(gate_mode == 1 || (A_log && dt_bias), "gdn_prefill_chunked: gate_mode 0 needs A_log, dt_bias");
    GDN_REQUIRE(cu_seqlens || T_total % N == 0, "gdn_prefill_chunked: T_total not divisible by N");
    GDN_REQUIRE(T_total < (int64_t(1) << 31), "gdn_prefill_chunked: token count must fit int32");
    GDN_REQUIRE(state_out, "gdn_prefill_chunked: null state_out");
    GDN_REQUIRE(T_total == 0 || (q && k && v && ga && gb && y), "gdn_prefill_chunked: null pointer");
    GDN_REQUIRE((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                 reinterpret_cast<uintptr_t>(state_in) | reinterpret_cast<uintptr_t>(state_out) |
                 reinterpret_cast<uintptr_t>(workspace)) % 16 == 0,
                "gdn_prefill_chunked: q, k, states and workspace must be 16-byte aligned");
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
    const int64_t L_uniform = cu_seqlens ? 0 : T_total / N;
    int32_t* chunk_off = static_cast<int32_t*>(workspace);
    char* records = static_cast<char*>(workspace) + records_offset(N);
    hipLaunchKernelGGL(chunk_offsets_kernel, dim3(1), dim3(64), 0, s, cu_seqlens, N, L_uniform, chunk_off);
    if (int rc = check_launch("gdn_prefill_chunked/offsets")) return rc;
    const int64_t nchunks = chunks_bound(T_total, N);
    hipLaunchKernelGGL(prefill_chunk_kernel, dim3(unsigned(nchunks), unsigned(Hk)), dim3(256), 0, s,
                       static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), ga, gb,
                       gb_dtype, A_log, dt_bias, gate_mode, cu_seqlens, N, L_uniform, chunk_off,
                       records, Hk, Hv);
    if (int rc = check_launch("gdn_prefill_chunked/chunk")) return rc;
    const dim3 sgrid(unsigned(int64_t(N) * Hv * kSlices));
#define GDN_STATE_LAUNCH(YT)                                                                      \
    hipLaunchKernelGGL(prefill_state_kernel<YT>, sgrid, dim3(256), 0, s,                          \
                       static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),           \
                       static_cast<const uint16_t*>(v), state_in, state_out,                       \
                       static_cast<YT::storage*>(y), cu_seqlens, N, L_uniform, chunk_off, records, \
                       Hk, Hv)
    if (y_dtype == GDN_F32) GDN_STATE_LAUNCH(ActF32);
    else if (y_dtype == GDN_BF16) GDN_STATE_LAUNCH(ActBF16);
    else GDN_STATE_LAUNCH(ActF16);
#undef GDN_STATE_LAUNCH
    return check_launch("gdn_prefill_chunked/state");
}
