/*
 * C restatement of the reference's gated-delta path, float32, OpenMP.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (as a second restatement that the
 * NumPy oracle must agree with) and by bench.py's cpu_baseline leg (the timed
 * CPU comparator, all host cores). Never part of the product path.
 *
 * Operation order follows the reference's pure-ops recurrence
 * (src/mlx_lean_moe/model/qwen3_5/gated_delta.py:35-39):
 *     state *= g; read = sum_k state*k; delta = (v - read)*beta;
 *     state += k*delta; y = sum_k state*q
 * with value head h reading key head h / (Hv/Hk) (gated_delta.py:99-101).
 * The decode step adds the layer's front-end and epilogue
 * (src/mlx_lean_moe/model/qwen3_5/linear_attention.py:22-32,61-79,109-124).
 * With act_bf16 != 0 values are rounded to bfloat16 where the reference holds
 * bf16 activations (same points as oracle/gated_delta_ref.py). The decode
 * step's front-end and gated norm evaluate each such value in double and
 * round it once; the recurrence itself runs in float32.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16r(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    memcpy(&x, &u, 4);
    return x;
}

static float rnd(float x, int act_bf16) { return act_bf16 ? bf16r(x) : x; }

/* One rounding of a double to the activation dtype: float32 by the cast;
 * bfloat16 by rounding the double's own mantissa to 8 significant bits
 * (nearest, ties to even), after which the cast to float is exact; below
 * 2^-126, bfloat16's subnormal range, to a multiple of 2^-133 (rint: ties to
 * even in the default rounding mode; the scalings are exact). The
 * front-end below evaluates each value the reference rounds to bf16 in
 * double and rounds it once, so a float32 error never decides a rounding
 * boundary (the float64 restatement in gated_delta_ref.py does the same). */
static float rnd_d(double x, int act_bf16) {
    if (!act_bf16) return (float)x;
    if (fabs(x) < 0x1p-126) return (float)(rint(x * 0x1p133) * 0x1p-133);
    uint64_t u;
    memcpy(&u, &x, 8);
    u = (u + ((1ull << 44) - 1) + ((u >> 45) & 1)) & ~((1ull << 45) - 1);
    memcpy(&x, &u, 8);
    return (float)x;
}

static double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

static float softplusf(float x) {
    /* logaddexp(x, 0) */
    float m = x > 0.f ? x : 0.f;
    return m + log1pf(expf(-fabsf(x)));
}

/* Sequential scan over L tokens for B sequences (uniform length).
 * q,k: (B, L, Hk, Dk); v: (B, L, Hv, Dv); g, beta: (B, L, Hv);
 * state_in/out: (B, Hv, Dv, Dk); y: (B, L, Hv, Dv). */
void gdn_ref_scan_f32(const float *q, const float *k, const float *v, const float *g,
                      const float *beta, const float *state_in, float *state_out, float *y,
                      int B, int L, int Hk, int Hv, int Dk, int Dv) {
    const int r = Hv / Hk;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int h = 0; h < Hv; ++h) {
            const int hk = h / r;
            float *S = state_out + ((size_t)b * Hv + h) * Dv * Dk;
            const float *S0 = state_in + ((size_t)b * Hv + h) * Dv * Dk;
            if (S != S0) memcpy(S, S0, sizeof(float) * Dv * Dk);
            for (int t = 0; t < L; ++t) {
                const size_t tok = (size_t)b * L + t;
                const float *qt = q + (tok * Hk + hk) * Dk;
                const float *kt = k + (tok * Hk + hk) * Dk;
                const float *vt = v + (tok * Hv + h) * Dv;
                const float gt = g[tok * Hv + h], bt = beta[tok * Hv + h];
                float *yt = y + (tok * Hv + h) * Dv;
                for (int i = 0; i < Dv; ++i) {
                    float *row = S + (size_t)i * Dk;
                    float read = 0.f;
                    for (int j = 0; j < Dk; ++j) row[j] *= gt;
                    for (int j = 0; j < Dk; ++j) read += row[j] * kt[j];
                    const float delta = (vt[i] - read) * bt;
                    float out = 0.f;
                    for (int j = 0; j < Dk; ++j) row[j] += kt[j] * delta;
                    for (int j = 0; j < Dk; ++j) out += row[j] * qt[j];
                    yt[i] = out;
                }
            }
        }
    }
}

/* One fused decode step for B sequences: conv(K taps)+SiLU+roll, q/k scaling,
 * gates, recurrence and (if z != NULL) the gated RMSNorm.
 * qkv: (B, C) pre-conv; conv_in/conv_out: (B, K-1, C); conv_w: (C, K);
 * a, b: (B, Hv); A_log, dt_bias: (Hv); state_in/out: (B, Hv, Dv, Dk);
 * z: (B, Hv, Dv) or NULL; norm_w: (Dv); out: (B, Hv, Dv). */
void gdn_ref_decode_f32(const float *qkv, const float *conv_in, float *conv_out,
                        const float *conv_w, const float *a, const float *bb,
                        const float *A_log, const float *dt_bias, const float *state_in,
                        float *state_out, const float *z, const float *norm_w, float eps,
                        float *out, int B, int Hk, int Hv, int Dk, int Dv, int K, int act_bf16) {
    const int C = 2 * Hk * Dk + Hv * Dv;
    const int r = Hv / Hk;
    const float inv = 1.f / sqrtf((float)Dk);
    const float sq = rnd(inv * inv, act_bf16), sk = rnd(inv, act_bf16);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int h = 0; h < Hv; ++h) {
            const int hk = h / r;
            float qv[256], kv[256], vv[256], yv[256];
            const float *x = qkv + (size_t)b * C;
            const float *cs = conv_in + (size_t)b * (K - 1) * C;
            /* conv over the channels this head reads */
            for (int part = 0; part < 3; ++part) {
                const int n = part < 2 ? Dk : Dv;
                const int base = part == 0 ? hk * Dk : part == 1 ? Hk * Dk + hk * Dk : 2 * Hk * Dk + h * Dv;
                float *dst = part == 0 ? qv : part == 1 ? kv : vv;
                for (int i = 0; i < n; ++i) {
                    const int c = base + i;
                    double acc = 0.0;
                    for (int j = 0; j < K; ++j) {
                        const float in = j < K - 1 ? rnd(cs[(size_t)j * C + c], act_bf16) : rnd(x[c], act_bf16);
                        acc += (double)rnd(conv_w[(size_t)c * K + j], act_bf16) * in;
                    }
                    const double cv = rnd_d(acc, act_bf16);
                    dst[i] = rnd_d(cv * sigmoid_d(cv), act_bf16);
                }
            }
            /* conv state roll: written once per channel (by the first value head of a key head for q/k) */
            float *co = conv_out + (size_t)b * (K - 1) * C;
            for (int part = 0; part < 3; ++part) {
                if (part < 2 && h % r != 0) continue;
                const int n = part < 2 ? Dk : Dv;
                const int base = part == 0 ? hk * Dk : part == 1 ? Hk * Dk + hk * Dk : 2 * Hk * Dk + h * Dv;
                for (int i = 0; i < n; ++i) {
                    const int c = base + i;
                    for (int j = 0; j < K - 1; ++j)
                        co[(size_t)j * C + c] = j + 1 < K - 1 ? rnd(cs[(size_t)(j + 1) * C + c], act_bf16) : rnd(x[c], act_bf16);
                }
            }
            double ssq = 0.0, ssk = 0.0;
            for (int i = 0; i < Dk; ++i) { ssq += (double)qv[i] * qv[i]; ssk += (double)kv[i] * kv[i]; }
            const double rq = 1.0 / sqrt(ssq / Dk + 1e-6), rk = 1.0 / sqrt(ssk / Dk + 1e-6);
            for (int i = 0; i < Dk; ++i) {
                qv[i] = rnd(sq * rnd_d(qv[i] * rq, act_bf16), act_bf16);
                kv[i] = rnd(sk * rnd_d(kv[i] * rk, act_bf16), act_bf16);
            }
            const float gt = expf(-expf(A_log[h]) * softplusf(a[(size_t)b * Hv + h] + dt_bias[h]));
            const float bt = rnd_d(sigmoid_d(bb[(size_t)b * Hv + h]), act_bf16);
            const float *S0 = state_in + ((size_t)b * Hv + h) * Dv * Dk;
            float *S = state_out + ((size_t)b * Hv + h) * Dv * Dk;
            if (S != S0) memcpy(S, S0, sizeof(float) * Dv * Dk);
            for (int i = 0; i < Dv; ++i) {
                float *row = S + (size_t)i * Dk;
                float read = 0.f, o = 0.f;
                for (int j = 0; j < Dk; ++j) row[j] *= gt;
                for (int j = 0; j < Dk; ++j) read += row[j] * kv[j];
                const float delta = (vv[i] - read) * bt;
                for (int j = 0; j < Dk; ++j) row[j] += kv[j] * delta;
                for (int j = 0; j < Dk; ++j) o += row[j] * qv[j];
                yv[i] = rnd(o, act_bf16);
            }
            float *ot = out + ((size_t)b * Hv + h) * Dv;
            if (z) {
                double ss = 0.0;
                for (int i = 0; i < Dv; ++i) ss += (double)yv[i] * yv[i];
                const double rr = 1.0 / sqrt(ss / Dv + (double)eps);
                const float *zt = z + ((size_t)b * Hv + h) * Dv;
                for (int i = 0; i < Dv; ++i) {
                    const double nrm = rnd_d(yv[i] * rr * norm_w[i], act_bf16);
                    const double zz = zt[i];
                    ot[i] = rnd_d(zz * sigmoid_d(zz) * nrm, act_bf16);
                }
            } else {
                for (int i = 0; i < Dv; ++i) ot[i] = yv[i];
            }
        }
    }
}

/* The one-rounding of a double to bfloat16 above, for the tests that pin it. */
float gdn_ref_bf16_of_double(double x) { return rnd_d(x, 1); }
