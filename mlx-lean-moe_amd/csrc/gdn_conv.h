// The bf16 prefill front-end's per-token arithmetic for eight channels of one
// 128-channel group (linear_attention.py:61-79,103-113): the causal K = 4
// conv, SiLU and the q/k scaling. Shared by the tiled front-end kernel and the
// fused chunk pass of the prefill, so that both produce the same bits. Every
// rounding is written out (fused multiply-adds where named, no other
// contraction), so that the two kernels round alike whatever code surrounds
// the calls.
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
#pragma clang fp contract(off)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float acc = wr[e][0] * win[0][e];
        acc = __builtin_fmaf(wr[e][1], win[1][e], acc);
        acc = __builtin_fmaf(wr[e][2], win[2][e], acc);
        o[e] = __builtin_fmaf(wr[e][3], x[e], acc);
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2) round_bf16x2(o[e], o[e + 1]);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = silu_hw(o[e]);
#pragma unroll
    for (int e = 0; e < 8; e += 2) round_bf16x2(o[e], o[e + 1]);
}

// rms_norm(o, 1e-6) of one token's 128-channel group held 8 channels a lane by
// the 16 lanes of a DPP row (every lane of the wave active), rounded to bf16.
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
