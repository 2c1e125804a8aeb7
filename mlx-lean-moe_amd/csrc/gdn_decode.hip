// Fused single-token decode for B sequences: one workgroup per
// (sequence, value head) runs the layer's whole per-token path between the
// projections (linear_attention.py:103-124):
//
//   conv(K=4) + SiLU over the head's q/k/v channels, conv-state roll,
//   q/k scaling, forget gate and beta, the gated-delta step, and (optionally)
//   the gated RMSNorm.
//
// The Dv x Dk = 128 x 128 float32 state tile (64 KiB) is the only large
// operand. Its 16 float4 loads per thread are issued first, so the HBM
// latency hides behind the front-end arithmetic; each row is then read once
// and written once, in 1 KiB-contiguous wave accesses (lanes 0-31 cover one
// 512-byte row, lanes 32-63 the next).
//
// Per thread (wave w, lane l, half = l / 32, l32 = l % 32) the tile rows are
// r_i = 8 i + 2 w + half, i = 0..15, columns 4 l32 .. 4 l32 + 3. The 32
// partial dot products a half-wave holds (S.k and S.q for its 16 rows) are
// reduce-scattered across the 32 lanes (31 exchanges instead of 160, all in
// registers: permlane swaps and DPP, no LDS round trip), which leaves lane
// l32 with the full S.k of row r_{l32} (l32 < 16) or the full S.q of row
// r_{l32-16} (l32 >= 16). Then
//     delta = beta (v - g S.k),   y = g S.q + delta (k.q),   S <- g S + delta k^T
// (the reference's decay/read/delta/update/output step, gated_delta.py:35-39,
// with the output taken from the pre-update row).
//
// Few sequences (B * Hv below 256 workgroups, a single sequence above all)
// leave most of the 256 CUs idle, so there a step without the gated norm
// gives each head kSplit workgroups (and from kPairSplitHeads heads on, two:
// two independently scheduled half-tile workgroups per head keep the HBM
// stream closer to its ceiling than one; one 512-thread workgroup holding
// both halves does not): split p reads, updates and stores rows
// [row0, row0 + 128 / kSplit), row0 = p * 128 / kSplit (rows r_i = row0 +
// 8 i + 2 w + half, i < 16 / kSplit, and a reduce-scatter over 32 / kSplit
// values per lane on the same butterfly). Each row's arithmetic is the
// one-workgroup path's, so state and y are the same bits. Every split
// recomputes the head's front-end (q, k and v are a few hundred channels);
// the first rolls the conv state. The norm needs the head's 128 outputs
// together: exchanging them between workgroups (a device-scope release and
// acquire each) costs more than the split saves, and reading the whole tile
// in every split races with the in-place update of the other splits' rows,
// so a step with the norm keeps one workgroup per head. With few heads
// (at most kSubHeads) that workgroup has kSub = 2 row blocks of 256 threads,
// each laid out as one workgroup of a two-way split (rows rb0 + 8 i + 2 w +
// half): twice the loads in flight per CU, one front-end, the head's outputs
// together in LDS for the norm.
#include "gdn_common.h"
#include "gdn_conv.h"
#include "gdn_host.h"

namespace gdn {

constexpr int kDecodeThreads = 256;
// What a step adds to a decoded slot's conv_arrivals counter, in equal
// shares over the row's workgroups (Hv * kSplit of them: a power of two).
constexpr int kArrivalStep = 1 << 16;
constexpr int kD = 128;   // Dk = Dv
constexpr int kTaps = 4;  // conv kernel K

#ifndef GDN_DECODE_NT
#define GDN_DECODE_NT 1
#endif

// Launches without the gated norm of at most kSplitGroups / 2 (sequence,
// head) pairs share each head among up to kMaxSplit workgroups (a power of
// two <= 16).
#ifndef GDN_DECODE_SPLIT_GROUPS
#define GDN_DECODE_SPLIT_GROUPS 256
#endif
#ifndef GDN_DECODE_MAX_SPLIT
#define GDN_DECODE_MAX_SPLIT 8
#endif
// From this many (sequence, head) pairs a step without the norm runs two
// workgroups per head (measured, Hv=32: B=64 49.3 -> 46.9 us, B=128 96.3 ->
// 91.4, B=256 186.0 -> 178.5; B=32 unchanged, smaller batches slower with
// more splits).
constexpr int64_t kPairSplitHeads = 2048;
// Up to this many heads a step with the norm runs 512-thread workgroups
// (measured, Hv=32: B=1 5.65 -> 5.39 us, B=8 8.58 -> 7.90; B=16 slower, and
// B=256, Hv=64 369 -> 389 us).
constexpr int64_t kSubHeads = 256;
constexpr int64_t kSplitGroups = GDN_DECODE_SPLIT_GROUPS;
constexpr int kMaxSplit = GDN_DECODE_MAX_SPLIT;
static_assert(kMaxSplit >= 1 && kMaxSplit <= 16 && (kMaxSplit & (kMaxSplit - 1)) == 0,
              "GDN_DECODE_MAX_SPLIT: 1, 2, 4, 8 or 16");

// The state is streamed exactly once per launch: optionally mark its loads
// and stores non-temporal.
GDN_DEV float4 load_state(const float4* p) {
#if GDN_DECODE_NT
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
#else
    return *p;
#endif
}

GDN_DEV void store_state(float4* p, float4 v) {
#if GDN_DECODE_NT
    const f32x4 x = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(x, reinterpret_cast<f32x4*>(p));
#else
    *p = v;
#endif
}

constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }

// One reduce-scatter level at partner distance OFF <= 8 over the first n of
// `vals`: a lane whose bit OFF is set keeps the upper half, the other lane of
// the pair the lower half, each adding the partner's copy of what it keeps.
template <int OFF, int n, int N>
GDN_DEV void scatter_level(float (&vals)[N], int l32) {
    const uint32_t upper = opaque_mask((l32 & OFF) != 0);
#pragma unroll
    for (int j = 0; j < n / 2; ++j) {
        const float keep = mask_select(upper, vals[j + n / 2], vals[j]);
        const float send = mask_select(upper, vals[j], vals[j + n / 2]);
        vals[j] = keep + dpp_partner<OFF>(send);
    }
}

// Sum `vals` (N <= 32 per lane, a power of two) over the 32 lanes of each
// half-wave on one butterfly, partners at levels 16, 8, 4, 2, 1 (lane pairings
// of group_sum): the first log2(N) levels also halve the values a lane
// carries (reduce-scatter), the rest add the one left (all-reduce). Lane l32
// ends with the total of index l32 >> (5 - log2(N)) in vals[0]. Both lanes of
// a pair add the same two partials, so every total is the same sum tree over
// the same 32 lane partials, bit for bit, whatever N is.
template <int N>
GDN_DEV void reduce_scatter(float (&vals)[N], int l32) {
    constexpr int kLevels = ilog2(N);
    static_assert(N >= 2 && N <= 32 && (N & (N - 1)) == 0, "2 to 32 values");
    // level 16: the swap leaves a lower-row lane its and its partner's lower
    // half, an upper-row lane the partner's and its upper half
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
        lane_swap<16>(vals[j], vals[j + N / 2]);
        vals[j] += vals[j + N / 2];
    }
    if constexpr (kLevels >= 2) scatter_level<8, N / 2>(vals, l32); else vals[0] = pair_sum<8>(vals[0]);
    if constexpr (kLevels >= 3) scatter_level<4, N / 4>(vals, l32); else vals[0] = pair_sum<4>(vals[0]);
    if constexpr (kLevels >= 4) scatter_level<2, N / 8>(vals, l32); else vals[0] = pair_sum<2>(vals[0]);
    if constexpr (kLevels >= 5) scatter_level<1, N / 16>(vals, l32); else vals[0] = pair_sum<1>(vals[0]);
}

// One conv channel's inputs: its K = 4 weights, the three conv-state taps and
// the current token.
struct ConvTaps {
    float4 w;
    float x0, x1, x2, x3;
};

template <class Act>
GDN_DEV ConvTaps load_taps(const typename Act::storage* __restrict__ x,
                           const typename Act::storage* __restrict__ cs,
                           const float4* __restrict__ w4, int C, int c) {
    return {w4[c], Act::load(cs, c), Act::load(cs, C + c), Act::load(cs, 2 * C + c),
            Act::load(x, c)};
}

// conv (cross-correlation, last tap on the current token) + SiLU, with the
// weights and the result held in the activation dtype: the prefill's conv
// chain (conv_chain: the same bits), and SiLU from libm's expf and an IEEE
// divide (within about two float ulps; the prefill's silu_hw, within about
// twenty, can round a value near a bf16 boundary the other way).
template <class Act>
GDN_DEV float conv_silu(const ConvTaps& t) {
    const float w[4] = {Act::round(t.w.x), Act::round(t.w.y), Act::round(t.w.z), Act::round(t.w.w)};
    const float x[4] = {t.x0, t.x1, t.x2, t.x3};
    const float acc = Act::round(conv_chain(4, [&](int j) { return float2{w[j], x[j]}; }));
    return Act::round(silu(acc));
}

// New conv state of a channel: the last K - 1 = 3 inputs.
template <class Act>
GDN_DEV void roll_taps(const ConvTaps& t, typename Act::storage* __restrict__ cso, int C, int c) {
    Act::store(cso, c, t.x1);
    Act::store(cso, C + c, t.x2);
    Act::store(cso, 2 * C + c, t.x3);
}

template <class Act, bool kNorm, int kSplit, int kSub = 1>
__global__ __launch_bounds__(kDecodeThreads * kSub) void decode_kernel(
    const typename Act::storage* __restrict__ qkv, const typename Act::storage* __restrict__ cs_in,
    typename Act::storage* __restrict__ cs_out, const float* __restrict__ conv_w,
    const typename Act::storage* __restrict__ a_in, const typename Act::storage* __restrict__ b_in,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias, const float* S_in,
    float* S_out, const typename Act::storage* __restrict__ z, const float* __restrict__ norm_w,
    float eps, void* __restrict__ out, int y_dtype, int Hk, int Hv,
    const int32_t* __restrict__ slots, int pool, int32_t* conv_half, int32_t* arrivals,
    int64_t qkv_stride, int64_t z_stride, int64_t a_stride, int64_t b_stride) {
    static_assert(kSplit >= 1 && kSplit <= 16 && (kSplit & (kSplit - 1)) == 0, "kSplit: 1, 2, 4, 8 or 16");
    static_assert(!kNorm || kSplit == 1, "the gated norm runs one workgroup per head");
    static_assert(kSub == 1 || (kSub == 2 && kSplit == 1), "kSub: 1, or 2 row blocks of a whole head");
    constexpr int kRows = kD / kSplit;        // state rows per workgroup
    constexpr int kR = 16 / (kSplit * kSub);  // state rows per thread
    constexpr int kN = 2 * kR;          // S.k and S.q partials per thread
    __shared__ float qs[kD], ks[kD], vs[kD], deltas[kD], ys[kD];
    __shared__ float gate_g, gate_beta;

    const int C = 2 * Hk * kD + Hv * kD;
    const int bh = blockIdx.x / kSplit;
    const int row0 = (blockIdx.x % kSplit) * kRows;  // this workgroup's first state row
    const bool first = row0 == 0;
    const int b = bh / Hv, h = bh % Hv;
    const int r = Hv / Hk, hk = h / r;
    const int tid = threadIdx.x;
    const int wg = tid >> 6;  // the wave in the workgroup
    // the thread's 256-thread row block: rows rb0 .. rb0 + kRows / kSub - 1
    const int t8 = kSub == 1 ? tid : tid & (kDecodeThreads - 1);
    const int rb0 = row0 + (kSub == 1 ? 0 : (tid >> 8) * (kRows / kSub));
    const int w = t8 >> 6, l = t8 & 63, half = l >> 5, l32 = l & 31;
    typename Act::storage* yo = static_cast<typename Act::storage*>(out);
    // the state slot of batch row b (its state tile is read and written
    // there) and its conv state rows (read at ci, rolled into co): the slot
    // and the batch row, or with conv_half the slot's current and other half
    // of a two-half array; the inputs are read at their row strides
    const int sl = slots ? slots[b] : b;
    if (unsigned(sl) >= unsigned(pool)) {  // a slot outside the pool: touch no state
        if (first && tid < kD)
            store_any(out, size_t(bh) * kD + tid, kNorm ? Act::code : y_dtype, __builtin_nanf(""));
        return;
    }
    int ci = sl, co = b;
    if (conv_half) {
        // with the counters, bit 16 of the slot's counter flips once per
        // step (kArrivalStep below): the half is the bit XOR that parity.
        // Plain loads: the launch's acquire makes earlier launches' atomics
        // visible, and a count read before other workgroups of this launch
        // add their shares has the same bit 16. (Agent-scope loads measured
        // ~0.1 us slower at one sequence.)
        const int hb = (conv_half[sl] ^ (arrivals ? arrivals[sl] >> 16 : 0)) & 1;
        ci = sl + pool * hb;
        co = sl + pool * (1 - hb);
    }
    const size_t sh = size_t(sl) * Hv + h;  // the state tile's index

    // A. the front-end's few inputs first, then the state loads: waiting for
    // the former does not wait for the latter.
    const typename Act::storage* x = qkv + b * qkv_stride;
    const typename Act::storage* cs = cs_in + size_t(ci) * (kTaps - 1) * C;
    typename Act::storage* cso = cs_out + size_t(co) * (kTaps - 1) * C;
    const float4* w4 = reinterpret_cast<const float4*>(conv_w);
    const int e = tid & (kD - 1);
    // pass 1: q channel (tid < 128) or k channel (tid >= 128) of key head hk;
    // pass 2: v channel of value head h (tid < 128).
    const int c1 = (tid < kD ? 0 : Hk * kD) + hk * kD + e;
    const int c2 = 2 * Hk * kD + h * kD + e;
    // (unconditional, so no branch forces a wait before the state loads)
    const ConvTaps t1 = load_taps<Act>(x, cs, w4, C, c1);
    const ConvTaps t2 = load_taps<Act>(x, cs, w4, C, c2);
    const float av = Act::load(a_in, b * a_stride + h), bv = Act::load(b_in, b * b_stride + h);
    const float alog = A_log[h], dtb = dt_bias[h];
    // the gated norm's gate and weight of this thread's output row (needed
    // last: loaded first, so no load waits at the end)
    float zz = 0.f, nw = 0.f;
    if (kNorm && tid < kD) {
        zz = Act::load(z, b * z_stride + h * kD + tid);
        nw = norm_w[tid];
    }

    const float4* Sb = reinterpret_cast<const float4*>(S_in + sh * kD * kD);
    float4 s[kR];
#pragma unroll
    for (int i = 0; i < kR; ++i) s[i] = load_state(&Sb[(rb0 + 8 * i + 2 * w + half) * (kD / 4) + l32]);

    // B. front-end for this head's channels (the first 256 threads).
    if (kSub == 1 || tid < 2 * kD) {
        (tid < kD ? qs : ks)[e] = conv_silu<Act>(t1);
        // q/k channels are shared by the r value heads of a key head: the first
        // workgroup of the first of them rolls their conv state.
        if (first && h % r == 0) roll_taps<Act>(t1, cso, C, c1);
    }
    // the two gates on two otherwise idle waves, in parallel
    if (tid < kD) {
        vs[e] = conv_silu<Act>(t2);
        if (first) roll_taps<Act>(t2, cso, C, c2);
    } else if (tid == kD) {
        gate_g = expf(log_forget_gate(av, alog, dtb));
    } else if (tid == kD + kWave) {
        gate_beta = beta_of(bv, Act::code);
    }
    __syncthreads();
    // Every thread has read the slot's half (its conv loads used it): thread
    // 0 adds this workgroup's share of the step's 2^16 to the slot's counter,
    // without waiting for the result. Bit 16 changes only with the last of
    // the row's Hv * kSplit shares, after every workgroup of the row has
    // read it, so the next launch reads the other half. (The form before,
    // where the last workgroup to count in flipped the bit and reset the
    // count, waited for the returned count and the flip: 0.7 us of a
    // one-sequence step, ~2 us at B=64.)
    if (arrivals && tid == 0)
        __hip_atomic_fetch_add(&arrivals[sl], kArrivalStep / (Hv * kSplit), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    if (wg < 2) {
        // rms_norm(x, 1e-6) rounded once from its exact value: the sum of
        // squares (exact in double for activation-dtype inputs), the
        // reciprocal root and the products in double (rms_rr); then the
        // scale, whose product with a 16-bit value is exact in float32. The
        // state's 1e-3 bound over chained steps needs q and k as the oracle
        // rounds them; the prefill's float32 rms_norm8 is within one bf16
        // ulp of these values
        float* arr = wg == 0 ? qs : ks;
        const float x0 = arr[l], x1 = arr[l + 64];
        const double rr = rms_rr(group_sum<kWave>(double(x0) * x0 + double(x1) * x1), kD);
        const float inv = 1.f / sqrtf(float(kD));
        const float sc = Act::round(wg == 0 ? inv * inv : inv);
        arr[l] = Act::round(sc * round_once(x0 * rr, Act::code));
        arr[l + 64] = Act::round(sc * round_once(x1 * rr, Act::code));
    }
    __syncthreads();

    // C. this lane's k and q slice, and k.q.
    const float4 kk = reinterpret_cast<const float4*>(ks)[l32];
    const float4 qq = reinterpret_cast<const float4*>(qs)[l32];
    const float kq = group_sum<32>(kk.x * qq.x + kk.y * qq.y + kk.z * qq.z + kk.w * qq.w);
    const float g = gate_g, beta = gate_beta;

    // D/E. partial dots, reduce-scattered over the half-wave.
    float vals[kN];
#pragma unroll
    for (int i = 0; i < kR; ++i) {
        vals[i] = s[i].x * kk.x + s[i].y * kk.y + s[i].z * kk.z + s[i].w * kk.w;
        vals[kR + i] = s[i].x * qq.x + s[i].y * qq.y + s[i].z * qq.z + s[i].w * qq.w;
    }
    reduce_scatter<kN>(vals, l32);

    // F. per-row delta (lanes < 16) and output (lanes >= 16); with kR < 16
    // rows, 16 / kR lanes hold each total and write the same value.
    {
        const int idx = l32 >> (5 - ilog2(kN));
        const int row = rb0 + 8 * (idx & (kR - 1)) + 2 * w + half;
        const float tot = vals[0];
        const float delta = (vs[row] - g * tot) * beta;
        float delta_pair = delta, unused = delta;  // lanes >= 16: the partner's delta
        lane_swap<16>(delta_pair, unused);
        if (l32 < 16) deltas[row] = delta;
        else ys[row] = g * tot + delta_pair * kq;
    }
    __syncthreads();
    // H. update and store the tile.
    float4* So = reinterpret_cast<float4*>(S_out + sh * kD * kD);
#pragma unroll
    for (int i = 0; i < kR; ++i) {
        const int row = rb0 + 8 * i + 2 * w + half;
        const float d = deltas[row];
        float4 o;
        o.x = g * s[i].x + d * kk.x;
        o.y = g * s[i].y + d * kk.y;
        o.z = g * s[i].z + d * kk.z;
        o.w = g * s[i].w + d * kk.w;
        store_state(&So[row * (kD / 4) + l32], o);
    }

    // I. output: y, or the gated RMSNorm of y held in the activation dtype.
    if (!kNorm) {
        if (tid < kRows) store_any(out, size_t(bh) * kD + row0 + tid, y_dtype, ys[row0 + tid]);
        return;
    }
    // the two output waves each reduce all 128 outputs (the same lanes, the
    // same order: the same bits), so no barrier hands the root between them
    if (tid < kD) {
        const float y0 = Act::round(ys[l]), y1 = Act::round(ys[l + 64]);
        const float ss = group_sum<kWave>(y0 * y0 + y1 * y1);
        const float nr = 1.f / sqrtf(ss / float(kD) + eps);
        const float yv = Act::round(ys[tid]);
        const float normed = Act::round(yv * nr * nw);
        Act::store(yo, size_t(bh) * kD + tid, silu(zz) * normed);
    }
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_decode_step(const void* qkv, const void* conv_state_in, void* conv_state_out,
                               const float* conv_weight, const void* a, const void* b,
                               const float* A_log, const float* dt_bias, const float* state_in,
                               float* state_out, const void* z, const float* norm_weight,
                               float norm_eps, void* out, int y_dtype, int B, int Hk, int Hv,
                               int Dk, int Dv, int K, int act_dtype, const int32_t* slots,
                               int pool, int32_t* conv_half, const int64_t* row_strides,
                               int32_t* conv_arrivals, void* stream) {
    GDN_REQUIRE(B >= 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0, "gdn_decode_step: bad head counts");
    GDN_REQUIRE(act_dtype == GDN_F32 || act_dtype == GDN_BF16,
                "gdn_decode_step: activations must be float32 or bfloat16");
    GDN_REQUIRE(valid_dtype(y_dtype), "gdn_decode_step: bad y dtype");
    if (Dk != kD || Dv != kD || K != kTaps)
        return fail(GDN_EUNSUPPORTED, "gdn_decode_step: specialised for Dk=Dv=128, K=4 (got %d, %d, %d)",
                    Dk, Dv, K);
    if (B == 0) return 0;
    GDN_REQUIRE(qkv && conv_state_in && conv_state_out && conv_weight && a && b && A_log &&
                    dt_bias && state_in && state_out && out,
                "gdn_decode_step: null pointer");
    GDN_REQUIRE(!z || norm_weight, "gdn_decode_step: z without norm_weight");
    if (!slots) pool = B;
    GDN_REQUIRE(pool >= 1, "gdn_decode_step: bad pool size %d", pool);
    GDN_REQUIRE(!conv_half || slots, "gdn_decode_step: conv_half needs slots");
    GDN_REQUIRE(!conv_arrivals || conv_half, "gdn_decode_step: conv_arrivals needs conv_half");
    if (conv_arrivals && ((Hv & (Hv - 1)) || Hv > kArrivalStep / 16))
        return fail(GDN_EUNSUPPORTED, "gdn_decode_step: conv_arrivals needs a power-of-two Hv up to %d (got %d)",
                    kArrivalStep / 16, Hv);
    const int64_t C = 2LL * Hk * kD + int64_t(Hv) * kD;
    const int64_t row_bytes = (kTaps - 1) * C * dtype_size(act_dtype);
    // with conv_half both conv pointers are the pool's two-half array (a
    // slot reads one half and writes the other); otherwise the two arrays
    // must not overlap
    if (conv_half)
        GDN_REQUIRE(conv_state_in == conv_state_out,
                    "gdn_decode_step: with conv_half, conv_state_in and conv_state_out are one array");
    else
        GDN_REQUIRE(!overlaps(conv_state_in, int64_t(pool) * row_bytes, conv_state_out, int64_t(B) * row_bytes),
                    "gdn_decode_step: conv_state_out overlaps conv_state_in");
    int64_t st[4] = {C, int64_t(Hv) * kD, Hv, Hv};  // qkv, z, a, b row strides
    if (row_strides)
        for (int i = 0; i < 4; ++i) {
            GDN_REQUIRE(row_strides[i] >= st[i], "gdn_decode_step: row stride %d is %lld, below %lld", i,
                        (long long)row_strides[i], (long long)st[i]);
            st[i] = row_strides[i];
        }
    const int64_t state_bytes = int64_t(pool) * Hv * kD * kD * 4;
    GDN_REQUIRE(state_in == state_out || !overlaps(state_in, state_bytes, state_out, state_bytes),
                "gdn_decode_step: state_out partially overlaps state_in");
    GDN_REQUIRE((reinterpret_cast<uintptr_t>(state_in) | reinterpret_cast<uintptr_t>(state_out) |
                 reinterpret_cast<uintptr_t>(conv_weight)) % 16 == 0,
                "gdn_decode_step: state and conv weight must be 16-byte aligned");
    // Below kSplitGroups workgroups a step without the norm shares each head
    // among up to kMaxSplit workgroups; from kPairSplitHeads heads, two.
    const int64_t heads = int64_t(B) * Hv;
    int split = 1;
    while (!z && split < kMaxSplit && heads * split * 2 <= kSplitGroups) split *= 2;
    if (!z && kMaxSplit >= 2 && heads >= kPairSplitHeads) split = 2;
    GDN_REQUIRE(heads * split <= INT32_MAX, "gdn_decode_step: B * Hv too large");
    const dim3 grid(unsigned(heads * split));
    const bool two_blocks = z && heads <= kSubHeads;  // the norm's workgroup: 512 threads
    hipStream_t s = as_stream(stream);
#define GDN_DECODE_LAUNCH(ACT, NORM, SPLIT, SUB)                                              \
    hipLaunchKernelGGL((decode_kernel<ACT, NORM, SPLIT, SUB>), grid, dim3(kDecodeThreads * SUB), 0, s, \
                       static_cast<const ACT::storage*>(qkv),                                 \
                       static_cast<const ACT::storage*>(conv_state_in),                       \
                       static_cast<ACT::storage*>(conv_state_out), conv_weight,               \
                       static_cast<const ACT::storage*>(a), static_cast<const ACT::storage*>(b), \
                       A_log, dt_bias, state_in, state_out, static_cast<const ACT::storage*>(z), \
                       norm_weight, norm_eps, out, y_dtype, Hk, Hv, slots, pool, conv_half,         \
                       conv_arrivals, st[0], st[1], st[2], st[3])
#define GDN_DECODE_SPLITS(ACT, NORM)                                   \
    switch (split) {                                                  \
        case 1: GDN_DECODE_LAUNCH(ACT, NORM, 1, 1); break;            \
        case 2: GDN_DECODE_LAUNCH(ACT, NORM, 2, 1); break;            \
        case 4: GDN_DECODE_LAUNCH(ACT, NORM, 4, 1); break;            \
        case 8: GDN_DECODE_LAUNCH(ACT, NORM, 8, 1); break;            \
        default: GDN_DECODE_LAUNCH(ACT, NORM, 16, 1); break;          \
    }
    if (act_dtype == GDN_BF16) {
        if (z && two_blocks) GDN_DECODE_LAUNCH(ActBF16, true, 1, 2);
        else if (z) GDN_DECODE_LAUNCH(ActBF16, true, 1, 1);
        else GDN_DECODE_SPLITS(ActBF16, false)
    } else {
        if (z && two_blocks) GDN_DECODE_LAUNCH(ActF32, true, 1, 2);
        else if (z) GDN_DECODE_LAUNCH(ActF32, true, 1, 1);
        else GDN_DECODE_SPLITS(ActF32, false)
    }
#undef GDN_DECODE_SPLITS
#undef GDN_DECODE_LAUNCH
    return check_launch("gdn_decode_step");
}

namespace gdn {
namespace {

__global__ void pool_advance_kernel(const int32_t* __restrict__ slots, int B, int32_t* __restrict__ half,
                                    int pool) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) {
        const int sl = slots[b];
        if (unsigned(sl) < unsigned(pool)) half[sl] ^= 1;
    }
}

}  // namespace
}  // namespace gdn

extern "C" int gdn_pool_advance(const int32_t* slots, int B, int32_t* conv_half, int pool, void* stream) {
    GDN_REQUIRE(B >= 0 && pool >= 1, "gdn_pool_advance: bad sizes");
    if (B == 0) return 0;
    GDN_REQUIRE(slots && conv_half, "gdn_pool_advance: null pointer");
    hipLaunchKernelGGL(pool_advance_kernel, dim3(unsigned((B + 255) / 256)), dim3(256), 0, as_stream(stream),
                       slots, B, conv_half, pool);
    return check_launch("gdn_pool_advance");
}

