// Shared device helpers for the gated-delta kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gdn.h"

#define GDN_DEV __device__ __forceinline__

namespace gdn {

constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// storage formats
// ---------------------------------------------------------------------------

// bfloat16 <-> float with round-to-nearest-even, done on the bit pattern so
// the rounding is exactly the one the CPU oracle applies.
GDN_DEV float bf16_bits_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// Round-to-nearest-even float32 -> bfloat16 (gfx950's v_cvt_pk_bf16_f32).
GDN_DEV uint16_t f32_to_bf16_bits(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }

GDN_DEV float round_bf16(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

GDN_DEV float f16_bits_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return float(v);
}

GDN_DEV uint16_t f32_to_f16_bits(float x) {
    _Float16 v = _Float16(x);
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// Eight bfloat16 values (16 bytes) <-> eight floats, element 0 in the low half
// of the first dword.
GDN_DEV void unpack8(uint4 r, float* x) {
    const uint32_t d[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(d[i] << 16);
        x[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
    }
}

// Two floats to two round-to-nearest-even bfloat16 in one dword (one
// v_cvt_pk_bf16_f32), a in the low half.
GDN_DEV uint32_t pack_bf16x2(float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// a and b rounded to bfloat16 precision, with one conversion for the pair.
GDN_DEV void round_bf16x2(float& a, float& b) {
    const uint32_t u = pack_bf16x2(a, b);
    a = __uint_as_float(u << 16);
    b = __uint_as_float(u & 0xFFFF0000u);
}

GDN_DEV uint4 pack8(const float* x) {
    return make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]),
                      pack_bf16x2(x[6], x[7]));
}

// Load element i of a buffer whose dtype is only known at run time (the
// branch is uniform across the wave).
GDN_DEV float load_any(const void* p, int64_t i, int dtype) {
    if (dtype == GDN_F32) return static_cast<const float*>(p)[i];
    const uint16_t h = static_cast<const uint16_t*>(p)[i];
    return dtype == GDN_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

GDN_DEV void store_any(void* p, int64_t i, int dtype, float x) {
    if (dtype == GDN_F32) {
        static_cast<float*>(p)[i] = x;
    } else {
        static_cast<uint16_t*>(p)[i] = dtype == GDN_BF16 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
    }
}

// Round a float32 value to what `dtype` can hold (identity for float32).
GDN_DEV float round_to(float x, int dtype) {
    if (dtype == GDN_F32) return x;
    return dtype == GDN_BF16 ? round_bf16(x) : f16_bits_to_f32(f32_to_f16_bits(x));
}

// One rounding of a double to what `dtype` holds: round to nearest even,
// as if from the exact value. float32 directly; bfloat16 and float16 through
// float32 rounded to odd (truncated, with the last bit set if anything was
// dropped), which keeps enough of the dropped bits for the second rounding
// to nearest to land where one rounding of the double would.
GDN_DEV float round_once(double x, int dtype) {
    if (dtype == GDN_F32) return float(x);
    float f = __double2float_rz(x);
    if (double(f) != x) f = __uint_as_float(__float_as_uint(f) | 1u);
    return round_to(f, dtype);
}

// beta = sigmoid(b) held in `dtype` (linear_attention.py:116): the value the
// exact sigmoid rounds to, so the decision at a rounding boundary does not
// depend on float32 error. For bfloat16 a float32 evaluation (within a few
// float ulps: expf, the sum, the reciprocal) decides it when it lies more
// than 16 float ulps from a bfloat16 rounding boundary (a low half-word of
// 0x8000; |b| < 64 keeps the value normal); otherwise, and for the other
// dtypes, the sigmoid is evaluated in double and rounded once.
GDN_DEV float beta_of(float b, int dtype) {
    if (dtype == GDN_BF16 && fabsf(b) < 64.f) {
        const float f = 1.f / (1.f + expf(-b));
        const uint32_t low = __float_as_uint(f) & 0xFFFFu;
        if (low + 16u < 0x8000u || low > 0x8000u + 16u) return round_bf16(f);
    }
    return round_once(1.0 / (1.0 + exp(-double(b))), dtype);
}

// Compile-time activation formats for the specialised kernels.
struct ActF32 {
    using storage = float;
    static constexpr int code = GDN_F32;
    static GDN_DEV float load(const storage* p, int64_t i) { return p[i]; }
    static GDN_DEV void store(storage* p, int64_t i, float x) { p[i] = x; }
    static GDN_DEV float round(float x) { return x; }
};

struct ActBF16 {
    using storage = uint16_t;
    static constexpr int code = GDN_BF16;
    static GDN_DEV float load(const storage* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
    static GDN_DEV void store(storage* p, int64_t i, float x) { p[i] = f32_to_bf16_bits(x); }
    static GDN_DEV float round(float x) { return round_bf16(x); }
};

struct ActF16 {
    using storage = uint16_t;
    static constexpr int code = GDN_F16;
    static GDN_DEV float load(const storage* p, int64_t i) { return f16_bits_to_f32(p[i]); }
    static GDN_DEV void store(storage* p, int64_t i, float x) { p[i] = f32_to_f16_bits(x); }
    static GDN_DEV float round(float x) { return f16_bits_to_f32(f32_to_f16_bits(x)); }
};

// ---------------------------------------------------------------------------
// math
// ---------------------------------------------------------------------------

// log(1 + e^x) in the logaddexp(x, 0) form (mlx.nn.softplus).
GDN_DEV float softplus(float x) { return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x))); }

GDN_DEV float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

GDN_DEV float silu(float x) { return x * sigmoid(x); }

// -exp(A_log) * softplus(a + dt_bias): log of the forget gate.
GDN_DEV float log_forget_gate(float a, float A_log, float dt_bias) {
    return -expf(A_log) * softplus(a + dt_bias);
}

// ---------------------------------------------------------------------------
// cross-lane reductions
// ---------------------------------------------------------------------------

// Per-lane choice between two values by an all-ones / all-zeros mask. The
// mask is hidden from the optimiser so that a choice between two elements of
// a register array is not rewritten into a dynamically indexed array.
GDN_DEV uint32_t opaque_mask(bool take_first) {
    uint32_t m = take_first ? 0xFFFFFFFFu : 0u;
    asm volatile("" : "+v"(m));
    return m;
}

GDN_DEV float mask_select(uint32_t m, float a, float b) {
    return __uint_as_float((__float_as_uint(a) & m) | (__float_as_uint(b) & ~m));
}

// Lane pairings without an LDS round trip. At level OFF (1, 2, 4, 8, 16, 32)
// the partner of lane l is l ^ 1 or l ^ 2 (DPP quad_perm), 7 - l within its
// 8 lanes (row_half_mirror), l ^ 8 within its 16 (row_ror:8), l ^ 16
// (v_permlane16_swap: rows 0 <-> 1, 2 <-> 3) or l ^ 32 (v_permlane32_swap).
// The partner always differs from l in bit log2(OFF) and agrees with it in
// every higher bit, so a butterfly over levels 1 .. WIDTH / 2 (or the other
// way round) reaches each lane of an aligned group of WIDTH exactly once.
// Every lane of the wave must be active.
template <int OFF>
constexpr int dpp_partner_ctrl() {
    static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8, "DPP levels: 1, 2, 4, 8");
    return OFF == 1 ? 0xB1 : OFF == 2 ? 0x4E : OFF == 4 ? 0x141 : 0x128;
}

// The partner lane's v, for OFF <= 8.
template <int OFF>
GDN_DEV float dpp_partner(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), dpp_partner_ctrl<OFF>(), 0xF, 0xF, false));
}

// The two operands of v_permlane16_swap / v_permlane32_swap (OFF = 16, 32)
// after the swap: a lane of the lower row (half) gets {its a, the partner's a},
// a lane of the upper one {the partner's b, its b}.
template <int OFF>
GDN_DEV void lane_swap(float& a, float& b) {
    static_assert(OFF == 16 || OFF == 32, "swap levels: 16, 32");
    const auto r = OFF == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false)
                             : __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

// x + the partner's x at level OFF: both lanes of a pair get the same bits.
template <int OFF>
GDN_DEV float pair_sum(float x) {
    if constexpr (OFF <= 8) {
        return x + dpp_partner<OFF>(x);
    } else {
        float a = x, b = x;
        lane_swap<OFF>(a, b);  // lower: {x_lower, x_upper}; upper: the same
        return a + b;
    }
}

template <int OFF>
GDN_DEV double pair_sum(double x) {
    float lo = __uint_as_float(uint32_t(__double_as_longlong(x)));
    float hi = __uint_as_float(uint32_t(uint64_t(__double_as_longlong(x)) >> 32));
    double other;
    if constexpr (OFF <= 8) {
        const uint64_t pl = __float_as_uint(dpp_partner<OFF>(lo)), ph = __float_as_uint(dpp_partner<OFF>(hi));
        other = __longlong_as_double(int64_t(pl | (ph << 32)));
    } else {
        float lo2 = lo, hi2 = hi;
        lane_swap<OFF>(lo, lo2);
        lane_swap<OFF>(hi, hi2);
        const double a = __longlong_as_double(int64_t(uint64_t(__float_as_uint(lo)) | (uint64_t(__float_as_uint(hi)) << 32)));
        const double b = __longlong_as_double(int64_t(uint64_t(__float_as_uint(lo2)) | (uint64_t(__float_as_uint(hi2)) << 32)));
        return a + b;
    }
    return x + other;
}

// Sum over each aligned group of WIDTH lanes (a power of two up to 64), the
// same bits in every lane of the group.
template <int WIDTH, class T>
GDN_DEV T group_sum(T x) {
    static_assert(WIDTH >= 1 && WIDTH <= kWave && (WIDTH & (WIDTH - 1)) == 0, "group width");
    if constexpr (WIDTH >= 2) x = pair_sum<1>(x);
    if constexpr (WIDTH >= 4) x = pair_sum<2>(x);
    if constexpr (WIDTH >= 8) x = pair_sum<4>(x);
    if constexpr (WIDTH >= 16) x = pair_sum<8>(x);
    if constexpr (WIDTH >= 32) x = pair_sum<16>(x);
    if constexpr (WIDTH >= 64) x = pair_sum<32>(x);
    return x;
}

// Sum over each row of 16 lanes, in every lane of the row, on DPP moves (no
// LDS round trip): pairs and quads (quad_perm), then the two quads of each
// half-row (row_half_mirror) and the two half-rows (row_mirror). Each step
// adds the same two values in every lane of a pair, so all 16 lanes end
// with the same bits.
GDN_DEV float row16_sum(float v) {
#define GDN_DPP_ADD(CTRL) \
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false))
    GDN_DPP_ADD(0xB1);   // quad_perm [1, 0, 3, 2]
    GDN_DPP_ADD(0x4E);   // quad_perm [2, 3, 0, 1]
    GDN_DPP_ADD(0x141);  // row_half_mirror
    GDN_DPP_ADD(0x140);  // row_mirror
#undef GDN_DPP_ADD
    return v;
}

// Index of the run that holds token t, given run offsets cu[0..n] (binary
// search; cu is non-decreasing, cu[0] = 0, cu[n] = T_total).
GDN_DEV int find_run(const int32_t* cu, int n, int64_t t) {
    int lo = 0, hi = n;  // invariant: cu[lo] <= t < cu[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cu[mid] <= t) lo = mid; else hi = mid;
    }
    return lo;
}

}  // namespace gdn
