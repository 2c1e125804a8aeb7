// The front-end's arithmetic (linear_attention.py:61-79,103-113): the causal
// conv, SiLU and the q/k scaling of the prefill's kernels (the tiled bf16
// front-end, the fused chunk pass, the general front-end), so that they
// produce the same bits. The conv chain (conv_chain) is the decode step's
// too. SiLU and the q/k scaling of 128-wide bf16 heads are float32
// (silu_hw, rms_norm8), each within a few float ulps of the exact value
// before its rounding to bf16: where that value lies nearer a bf16 rounding
// boundary, the result can differ by one bf16 ulp from the decode step's,
// which rounds the q/k scaling once from double and takes SiLU from expf and
// an IEEE divide. Every rounding is written out (fused multiply-adds where
// named, no other contraction).
#pragma once

#include "gdn_common.h"

namespace gdn {

// silu(x) = x / (1 + e^-x) on the hardware exp2 and reciprocal (about 1 ulp
// each; the argument's rounding adds under 2^-20 relative for |x| < 16):
// five instructions against about twenty-five for libm's expf and an IEEE
// divide, and within a few float ulp of them, far below the bf16 rounding
// the result gets next.
GDN_DEV float silu_hw(float x) {
#pragma clang fp contract(off)
    return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.44269504088896341f));
}

// SiLU of a value held in the activation dtype kDt, before its rounding to
// kDt: for bf16 silu_hw from -16 up (its rounding hides silu_hw's few float
// ulps; below -16 e^-x outgrows what exp2 and the reciprocal keep, and
// from about -87 on overflows them while silu(x) is still a bf16 value),
// else libm's expf and an IEEE divide (silu), as for float32 and float16.
// The redo below -16 is taken by a wave only when one of its values needs
// it (a select would evaluate both forms everywhere); each value's result
// depends on the value alone.
template <int kDt, int N>
GDN_DEV void silu_act(float (&x)[N]) {
    if constexpr (kDt == GDN_BF16) {
        bool low = false;
#pragma unroll
        for (int e = 0; e < N; ++e) low = low || x[e] < -16.f;
        float y[N];
#pragma unroll
        for (int e = 0; e < N; ++e) y[e] = silu_hw(x[e]);
        if (__builtin_amdgcn_ballot_w64(low) != 0) {
#pragma unroll
            for (int e = 0; e < N; ++e)
                if (x[e] < -16.f) y[e] = silu(x[e]);
        }
#pragma unroll
        for (int e = 0; e < N; ++e) x[e] = y[e];
    } else {
#pragma unroll
        for (int e = 0; e < N; ++e) x[e] = silu(x[e]);
    }
}

// The causal conv of one channel over K taps, sum_j w_j x_j in tap order
// (tap(j) gives (w_j, x_j)): the first product, then a chain of fused
// multiply-adds, before its rounding to the activation dtype.
template <class Tap>
GDN_DEV float conv_chain(int K, Tap tap) {
#pragma clang fp contract(off)
    float2 t = tap(0);
    float acc = t.x * t.y;
    for (int j = 1; j < K; ++j) {
        t = tap(j);
        acc = __builtin_fmaf(t.x, t.y, acc);
    }
    return acc;
}

// The q/k scaling's reciprocal root in double from the sum of squares ss
// (double; the squares of 16-bit values are exact) of D values:
// 1 / sqrt(ss / D + 1e-6). The scaled value x * rr is rounded once to the
// activation dtype (round_once): the oracle's evaluation.
GDN_DEV double rms_rr(double ss, int D) { return rsqrt(ss / double(D) + 1e-6); }

// Eight consecutive conv-state values at element `at`, rounded to bf16 (the
// state may be held in any float dtype; `at` is a multiple of 8, the buffer
// 16-byte aligned).
template <int kDt>
GDN_DEV void load_state8(const void* __restrict__ p, int64_t at, float* x) {
    if constexpr (kDt == GDN_F32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + at);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + at + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = round_bf16(v[e]);
    } else if constexpr (kDt == GDN_BF16) {
        unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + at), x);
    } else {
        const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + at);
        const uint32_t d[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = round_bf16(f16_bits_to_f32(uint16_t(d[i] & 0xFFFF)));
            x[2 * i + 1] = round_bf16(f16_bits_to_f32(uint16_t(d[i] >> 16)));
        }
    }
}

// The K = 4 taps of channels c0 .. c0 + 7 (float32 (C, 4), 16-byte rows),
// rounded to bf16 as the reference's bf16 conv weight holds them.
GDN_DEV void load_conv_w8(const float* __restrict__ w, int64_t c0, float (&wr)[8][4]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float4 v4 = *reinterpret_cast<const float4*>(w + (c0 + e) * 4);
        wr[e][0] = round_bf16(v4.x);
        wr[e][1] = round_bf16(v4.y);
        wr[e][2] = round_bf16(v4.z);
        wr[e][3] = round_bf16(v4.w);
    }
}

// One token of eight channels: the conv over rows t-3 .. t-1 (win) and row t
// (x), rounded to bf16, then SiLU, rounded to bf16.
GDN_DEV void conv_silu8(const float (&wr)[8][4], const float (&win)[3][8], const float (&x)[8],
                        float (&o)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float xs[4] = {win[0][e], win[1][e], win[2][e], x[e]};
        o[e] = conv_chain(4, [&](int j) { return float2{wr[e][j], xs[j]}; });
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2) round_bf16x2(o[e], o[e + 1]);
    silu_act<GDN_BF16>(o);
#pragma unroll
    for (int e = 0; e < 8; e += 2) round_bf16x2(o[e], o[e + 1]);
}

// rms_norm(o, 1e-6) of one token's 128-channel group held 8 channels a lane by
// the 16 lanes of a DPP row (every lane of the wave active), rounded to bf16:
// float32 throughout (twelve roundings of positive terms in the sum of
// squares, rsq within 1 ulp, the product: within 10 float ulps of the exact
// value before the rounding to bf16; rows whose squares overflow or
// underflow float32, |x| beyond about 1.8e19 or below 1e-19 throughout, are
// outside its range).
GDN_DEV void rms_norm8(const float (&o)[8], float (&n)[8]) {
#pragma clang fp contract(off)
    float ss = o[0] * o[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) ss = __builtin_fmaf(o[e], o[e], ss);
    const float r = __builtin_amdgcn_rsqf(row16_sum(ss) * (1.f / 128.f) + 1e-6f);
#pragma unroll
    for (int e = 0; e < 8; ++e) n[e] = o[e] * r;
#pragma unroll
    for (int e = 0; e < 8; e += 2) round_bf16x2(n[e], n[e + 1]);
}

}  // namespace gdn
