/*
 * gdn.h - C ABI of the MI355X (gfx950) gated-delta linear-attention library.
 *
 * The library replaces, on an AMD GPU, the kernel side of the reference's
 * gated-delta path (mlx-lean-moe, paths relative to its root):
 *
 *   src/mlx_lean_moe/model/qwen3_5/_gated_delta_metal.py:35-114  Metal scan kernel
 *   src/mlx_lean_moe/model/qwen3_5/gated_delta.py:14-109         gates, step, scan
 *   src/mlx_lean_moe/model/qwen3_5/linear_attention.py:22-124    conv front-end,
 *                                                                 q/k scaling, gated norm
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are device pointers to caller-allocated, densely
 *     packed (row-major, last axis contiguous) buffers. The library never
 *     allocates or frees device memory.
 *   - Sizes are plain ints / int64; dtypes are gdn_dtype codes.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL is the
 *     null stream) and is asynchronous; calls on different streams are
 *     independent (no mutable global state).
 *   - Return value: 0 on success, GDN_EINVAL (< 0) for an invalid argument
 *     (nothing is launched), GDN_EUNSUPPORTED (< 0) for a valid call this
 *     kernel does not specialise, or a positive hipError_t from the launch.
 *     gdn_last_error() returns a message for the calling thread's last
 *     failure.
 *   - Inputs are never written unless an output pointer aliases them where a
 *     function says aliasing is allowed.
 */
#ifndef GDN_H
#define GDN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    GDN_F32 = 0,
    GDN_BF16 = 1,
    GDN_F16 = 2
} gdn_dtype;

#define GDN_OK 0
#define GDN_EINVAL (-1)
#define GDN_EUNSUPPORTED (-2)

/* Library ABI version (bumped on any signature change or addition; 2 adds the
 * quantized matmul and dequantize entry points, 3 the decode step's state
 * slots, 4 its conv rows, 5 replaces the conv rows with the pool's half bits,
 * adds input row strides and gdn_pool_advance, 6 the quantized matmul's
 * workspace and the decode step's conv_arrivals, 7 the quantized matmul's
 * residual, 8 the prefill's gate row stride, 9 the front-end's qkv row stride,
 * 10 the gated norm's z layout, 11 gdn_quantized_matmul_noalloc, 12 the
 * prefill's float32 q/k/v, 13 gdn_prefill_fused, 14 gdn_dequantize's mode, 15
 * gdn_quantized_matmul_scheme and its workspace size, 16 conv_arrivals as
 * counters whose bit 16 is a parity of the half bit). */
int gdn_abi_version(void);

/* Message describing the calling thread's last non-zero return. */
const char *gdn_last_error(void);

/*
 * gdn_gates - per-(row, value-head) decay and write strength.
 *   g[i,h]    = exp(-exp(A_log[h]) * softplus(a[i,h] + dt_bias[h]))   (float32)
 *   beta[i,h] = sigmoid(b[i,h]) rounded to beta_dtype
 * a, b: (rows, Hv) in ab_dtype; A_log, dt_bias: (Hv) float32. Either output
 * may be NULL (then its inputs may be NULL too).
 * Replaces forget_gate (gated_delta.py:14-21) and mx.sigmoid(b)
 * (linear_attention.py:116).
 */
int gdn_gates(const void *a, const void *b, int ab_dtype, const float *A_log,
              const float *dt_bias, float *g, void *beta, int beta_dtype, int64_t rows,
              int Hv, void *stream);

/*
 * gdn_frontend - causal depthwise conv (K taps) + SiLU + conv-state roll and
 * q/k scaling for a batch of token runs.
 *   qkv:            (T_total, C) act_dtype, C = 2*Hk*Dk + Hv*Dv, channel order [q; k; v],
 *                   rows qkv_stride elements apart (>= C; C when packed: qkv may be
 *                   the first columns of a stacked projection output)
 *   conv_state_in:  (N, K-1, C) conv_dtype
 *   conv_state_out: (N, K-1, C) act_dtype (the reference keeps the rolled state in
 *                   the activation dtype); must not overlap conv_state_in
 *   conv_weight:    (C, K) float32 (the reference's (C, K, 1)); rounded to act_dtype
 *   cu_seqlens:     (N+1) int32 token offsets of the N runs, or NULL for N runs of
 *                   T_total/N tokens each
 *   q_out, k_out:   (T_total, Hk, Dk) act_dtype;  v_out: (T_total, Hv, Dv) act_dtype
 * q = Dk^-1 * rms_norm(q, 1e-6), k = Dk^-1/2 * rms_norm(k, 1e-6).
 * Replaces Qwen3_5LinearAttention._convolve and the split/scale
 * (linear_attention.py:61-79,103-113).
 */
int gdn_frontend(const void *qkv, int64_t qkv_stride, const void *conv_state_in, void *conv_state_out,
                 int conv_dtype, const float *conv_weight, const int32_t *cu_seqlens, int N,
                 int64_t T_total, void *q_out, void *k_out, void *v_out, int Hk, int Hv, int Dk,
                 int Dv, int K, int act_dtype, void *stream);

/*
 * gdn_scan_reference - plain sequential recurrence, one thread per state row,
 * the reference's operation order (gated_delta.py:35-39). Any Dk/Dv, any
 * dtype mix; arithmetic in float32. A test aid and the use_kernel=False path.
 *   q, k: (T_total, Hk, Dk); v: (T_total, Hv, Dv); g, beta: (T_total, Hv)
 *   state_in: (N, Hv, Dv, Dk) state_dtype; state_out: same (may alias state_in)
 *   y: (T_total, Hv, Dv) y_dtype
 *   cu_seqlens: (N+1) int32 or NULL (N runs of T_total/N tokens)
 * Replaces _gated_delta_scan_ops (gated_delta.py:93-109).
 */
int gdn_scan_reference(const void *q, const void *k, int qk_dtype, const void *v, int v_dtype,
                       const void *g, int g_dtype, const void *beta, int beta_dtype,
                       const void *state_in, void *state_out, int state_dtype, void *y,
                       int y_dtype, const int32_t *cu_seqlens, int N, int64_t T_total, int Hk,
                       int Hv, int Dk, int Dv, void *stream);

/*
 * gdn_scan - sequential recurrence with the state held in registers across
 * the token loop: 32 lanes per state row, 8 rows per workgroup. Same
 * arguments and layout as gdn_scan_reference; Dk in {32, 64, 128, 256}.
 * Replaces the Metal kernel lean_moe_gated_delta_scan_f32
 * (_gated_delta_metal.py:35-114), generalised to a batch of runs and to
 * bf16/f16 inputs.
 */
int gdn_scan(const void *q, const void *k, int qk_dtype, const void *v, int v_dtype,
             const void *g, int g_dtype, const void *beta, int beta_dtype,
             const void *state_in, void *state_out, int state_dtype, void *y, int y_dtype,
             const int32_t *cu_seqlens, int N, int64_t T_total, int Hk, int Hv, int Dk, int Dv,
             void *stream);

/*
 * gdn_decode_step - one fused decode token for B sequences: conv + SiLU +
 * conv-state roll, q/k scaling, gates, the recurrence, and optionally the
 * gated RMSNorm. One workgroup per (sequence, value head) (with the norm and
 * B * Hv at most 256, of 512 threads), or, without the norm, 2-8 workgroups
 * per head when B * Hv is at most 128 and 2 from B * Hv = 2048, each taking
 * a share of its rows (the same arithmetic per row: the same state and
 * output bits); the float32 Dv x Dk state tile is read once and written once.
 *   qkv:            (B, C) act_dtype (pre-conv projection output)
 *   conv_state_in:  (B, K-1, C) act_dtype; conv_state_out must not overlap it
 *   conv_weight:    (C, K) float32
 *   a, b:           (B, Hv) act_dtype;  A_log, dt_bias: (Hv) float32
 *   state_in:       (B, Hv, Dv, Dk) float32; state_out may alias state_in
 *   z:              (B, Hv, Dv) act_dtype or NULL; norm_weight: (Dv) float32
 *   out:            (B, Hv, Dv): act_dtype (gated-norm output) when z != NULL,
 *                   else the recurrence output y in y_dtype
 *   slots:          NULL (row b is state slot b), or (B) int32 distinct slot
 *                   indices into a pool of `pool` sequences: state_in/state_out
 *                   are (pool, Hv, Dv, Dk) and the tile of slots[b] is read and
 *                   written (pass state_out == state_in); without conv_half,
 *                   conv_state_in is (pool, K-1, C) read at slots[b] and
 *                   conv_state_out (B, K-1, C) written at row b (the caller
 *                   copies it back). pool is ignored when slots is NULL.
 *   conv_half:      NULL, or (pool) int32 (needs slots): the pool's conv state
 *                   is one (2 pool, K-1, C) array of two halves, passed as both
 *                   conv_state_in and conv_state_out; slot s holds its current
 *                   state at row s + pool * h(s) and row b rolls it into the
 *                   other half, row s + pool * (1 - h(s)), where h(s) is
 *                   conv_half[s] & 1 (XOR bit 16 of conv_arrivals[s] when the
 *                   counters are given). Without conv_arrivals the bits are only
 *                   read (gdn_pool_advance flips them after the step).
 *   row_strides:    NULL (dense inputs), or host int64[4]: the row strides, in
 *                   elements, of qkv, z, a and b (each at least its row width
 *                   C, Hv * Dv, Hv, Hv), so that slices of one stacked
 *                   projection output are read in place.
 *   conv_arrivals:  NULL, or (pool) int32 counters, zero at first (needs
 *                   conv_half and a power-of-two Hv): the step adds 2^16 to the
 *                   counter of each decoded slot (in equal shares over the
 *                   row's workgroups, so bit 16 flips when the last of them has
 *                   read the half), which flips h(s), so no gdn_pool_advance
 *                   follows. The bits below 16 are zero between calls. A pool
 *                   whose steps pass the counters must pass them on every step
 *                   (a step without them would read conv_half alone).
 *   A row whose slot falls outside the pool writes NaN to its output and
 *   touches no state.
 * Specialised for Dk = Dv = 128, K = 4; act_dtype in {F32, BF16}.
 * Replaces one decode call of Qwen3_5LinearAttention.__call__ between the
 * projections (linear_attention.py:103-124) with the Metal scan at T=1.
 */
int gdn_decode_step(const void *qkv, const void *conv_state_in, void *conv_state_out,
                    const float *conv_weight, const void *a, const void *b,
                    const float *A_log, const float *dt_bias, const float *state_in,
                    float *state_out, const void *z, const float *norm_weight, float norm_eps,
                    void *out, int y_dtype, int B, int Hk, int Hv, int Dk, int Dv, int K,
                    int act_dtype, const int32_t *slots, int pool, int32_t *conv_half,
                    const int64_t *row_strides, int32_t *conv_arrivals, void *stream);

/*
 * gdn_pool_advance - flip conv_half[slots[b]] for b < B: the slots decoded by
 * a gdn_decode_step call with conv_half now hold their conv state in the
 * other half. Slots outside [0, pool) are skipped; slots must be distinct.
 * One launch on `stream`, so a captured decode step includes it. Replaces the
 * cache update after a decode step (cache/recurrent_cache.py:24-41).
 */
int gdn_pool_advance(const int32_t *slots, int B, int32_t *conv_half, int pool, void *stream);

/*
 * gdn_prefill_chunked - chunked (WY/UT, 64-token chunks) prefill on bf16
 * MFMA with float32 accumulation, for N packed runs.
 *   q, k: (T_total, Hk, Dk);  v: (T_total, Hv, Dv), all in qkv_dtype:
 *         GDN_BF16 (used as they are) or GDN_F32 (each value split into a
 *         bf16 high part and a bf16 residual, the residual products added)
 *   gate_mode 0: ga = a, gb = b, both (T_total, Hv) in gb_dtype, with A_log and
 *                dt_bias (Hv) float32 (gates computed in-kernel, beta held in gb_dtype)
 *   gate_mode 1: ga = g (T_total, Hv) float32, gb = beta (T_total, Hv) gb_dtype
 *   gate_stride: elements between consecutive tokens' rows of ga and gb (>= Hv;
 *                Hv when packed), so a and b may be column slices of one
 *                projection output
 *   state_in: (N, Hv, Dv, Dk) float32 or NULL (zero state); state_out: (N, Hv, Dv, Dk),
 *             not aliasing state_in
 *   q, k, states and workspace 16-byte aligned, v 8-byte aligned (16 with
 *   float32 input)
 *   y: (T_total, Hv, Dv) y_dtype
 *   workspace: device scratch of gdn_prefill_workspace_size(...) bytes
 * Specialised for Dk = Dv = 128. Equal, up to rounding, to gdn_scan on the
 * same inputs. No reference counterpart: the reference prefills with the
 * sequential scan (_gated_delta_metal.py:64-87).
 */
int64_t gdn_prefill_workspace_size(int N, int64_t T_total, int Hk, int Hv, int Dk, int Dv);
int gdn_prefill_chunked(const void *q, const void *k, const void *v, int qkv_dtype, const void *ga,
                        const void *gb, int gb_dtype, int64_t gate_stride, const float *A_log,
                        const float *dt_bias, int gate_mode, const float *state_in,
                        float *state_out, void *y, int y_dtype, const int32_t *cu_seqlens,
                        int N, int64_t T_total, int Hk, int Hv, int Dk, int Dv, void *workspace,
                        int64_t workspace_bytes, void *stream);

/*
 * gdn_prefill_fused - the layer's prefill between the projections, short of
 * the gated norm: the front-end (conv + SiLU + conv-state roll, q/k scaling,
 * as gdn_frontend computes them, to the bit) and the chunked prefill, the
 * front-end done inside the chunk pass (q, k and v go to the workspace for
 * the state pass only). For N packed runs, bf16 activations.
 *   qkv: (T_total, C) bfloat16 rows at qkv_stride elements (>= C, a multiple
 *        of 8), C = (2 Hk + Hv) Dk
 *   conv_state_in: (N, K-1, C) conv_dtype (GDN_BF16 or GDN_F32);
 *   conv_state_out: (N, K-1, C) bfloat16, not overlapping conv_state_in
 *   conv_weight: (C, K) float32
 *   a, b: (T_total, Hv) gate_dtype at gate_stride (>= Hv) elements per token;
 *         A_log, dt_bias: (Hv) float32 (the gates as gdn_prefill_chunked's
 *         gate_mode 0)
 *   state_in: (N, Hv, Dv, Dk) float32 or NULL (zero); state_out: the same,
 *             not aliasing state_in
 *   y: (T_total, Hv, Dv) y_dtype
 *   workspace: device scratch of gdn_prefill_fused_workspace_size(...) bytes
 *   qkv, conv states, conv weight, states and workspace 16-byte aligned.
 * Specialised for Dk = Dv = 128, K = 4. Replaces the layer's conv and
 * gated_delta_update for a prompt (linear_attention.py:103-121), with the
 * same results as gdn_frontend followed by gdn_prefill_chunked.
 */
int64_t gdn_prefill_fused_workspace_size(int N, int64_t T_total, int Hk, int Hv, int Dk, int Dv);
int gdn_prefill_fused(const void *qkv, int64_t qkv_stride, const void *conv_state_in,
                      void *conv_state_out, int conv_dtype, const float *conv_weight, int K,
                      const void *a, const void *b, int gate_dtype, int64_t gate_stride,
                      const float *A_log, const float *dt_bias, const float *state_in,
                      float *state_out, void *y, int y_dtype, const int32_t *cu_seqlens, int N,
                      int64_t T_total, int Hk, int Hv, int Dk, int Dv, void *workspace,
                      int64_t workspace_bytes, void *stream);

/*
 * gdn_gated_rmsnorm - out = silu(z) * rms_norm(x, w, eps) with x first rounded
 * to out_dtype and the normalised value held in out_dtype; the product is
 * taken in float32 and stored in out_dtype.
 *   x: (rows, D) x_dtype; w: (D) float32; out: (rows, D) out_dtype
 *   z: rows of D z_dtype elements, row r at element (r / heads) * z_stride +
 *      (r % heads) * D (heads = 1, z_stride = D when packed; the layer's
 *      (T, Hv, D) column view of a stacked projection output: heads = Hv and
 *      z_stride its token stride); rows % heads == 0, z_stride >= heads * D
 * Replaces _gated_rms_norm (linear_attention.py:22-32); with out_dtype = z's
 * dtype it includes its call site's y.astype(z.dtype) (linear_attention.py:122-124).
 */
int gdn_gated_rmsnorm(const void *x, int x_dtype, const void *z, int z_dtype, int64_t z_stride,
                      int heads, const float *w, float eps, void *out, int out_dtype, int64_t rows,
                      int D, void *stream);

/*
 * gdn_quantized_matmul - y = x W^T for an affine-quantized W in MLX's packing,
 * on bf16 MFMA with float32 accumulation.
 *   x: (M, K) bfloat16; or float32 with M <= 32 on the decode kernel's shapes,
 *      staged as bf16 hi + lo (~16 significant bits; other cases:
 *      GDN_EUNSUPPORTED, see gdn_dequantize)
 *   w: (N, K * bits / 32) uint32, element k of row n at bits [bits * (k % (32 / bits)), +bits)
 *      of word k / (32 / bits), least significant first; 16-byte aligned
 *   scales, biases: (N, K / group_size) sb_dtype; w[n][k] = scales[n][g] * q + biases[n][g]
 *   y: (M, N) y_dtype
 *   bits 4 or 8 (others: GDN_EUNSUPPORTED); group_size 32, 64 or 128; K a
 *   multiple of 64 and of group_size
 * Up to 64 rows, on the shapes the decode kernel takes (decode_kernel_fits in
 * gdn_qlinear.hip: K in whole steps of 8 quantization slices, K / group_size
 * <= 64, 16-byte aligned operands; the layer's projections at hidden 2048 and
 * value dim 4096 all qualify): products against the exact weights
 * scale * q + bias, with scale
 * and bias applied per group to float partial sums (as MLX's matrix-vector
 * kernels do). Otherwise the weights enter the MFMAs as bf16(scale * q + bias)
 * (the product is exact in float32; one rounding), i.e. x times the weights
 * mx.dequantize yields (as MLX's matrix-matrix kernels do).
 *   residual: NULL, or (M, N) y_dtype (may be y itself): y = the product
 *      rounded to y_dtype plus residual, rounded again (the unfused add of
 *      two y_dtype arrays, as the decoder layer's h = x + attention(...),
 *      model/qwen3_5/transformer.py:110-112)
 *   workspace: NULL, or device scratch of workspace_bytes (16-byte aligned).
 *      With gdn_quantized_matmul_workspace_size(...) bytes, a decode-kernel
 *      call with few column tiles (small N) splits K over several
 *      workgroups, which store float32 partial products there, and a second
 *      kernel adds them in a fixed order (deterministic; the sum's order,
 *      and so its last bits, differ from the unsplit kernel's). With less,
 *      it splits less or not at all. 17-64 rows of bf16 x against 4-bit
 *      codes in 64-k slices with few column tiles (out_proj's shape) run
 *      instead as 16-row blocks in one launch and take no workspace (its
 *      size is 0 there). Calls sharing a workspace must not overlap.
 * Replaces mx.quantized_matmul(..., mode="affine") in quantized_linear
 * (model/moe_block.py:44-55), used for the layer's projections
 * (model/qwen3_5/linear_attention.py:96-101,125).
 */
int gdn_quantized_matmul(const void *x, int x_dtype, const void *w, const void *scales,
                         const void *biases, int sb_dtype, void *y, int y_dtype,
                         const void *residual, int M, int N, int K, int bits, int group_size,
                         void *workspace, int64_t workspace_bytes, void *stream);

/*
 * gdn_quantized_matmul_noalloc - gdn_quantized_matmul that allocates nothing
 * and takes no workspace: a call that splits K keeps its float32 partial
 * products in the library's own device scratch (a static 4 MiB array per
 * GPU, held until the process ends; every call the decode kernel takes
 * needs at most that), so it splits exactly as gdn_quantized_matmul does
 * with a full workspace and gives the same bits. A call needing more
 * returns GDN_EINVAL. The first call on a GPU looks up that GPU's copy of
 * the array (hipGetSymbolAddress, which may load the library's code object
 * there): make that first call eagerly, before capturing calls into a HIP
 * graph on that GPU (that call also creates the GPU's one ordering
 * event). No call allocates or frees memory. The calls that use the
 * scratch take it in turn: one on a different stream than the previous
 * scratch user first makes its stream wait (hipStreamWaitEvent) for that
 * call, so calls from several streams and host threads do not race. A call
 * made while its stream is being captured neither waits nor records (a
 * capture cannot wait on work outside it): replays of such a graph are
 * ordered against calls on other streams by the caller. Arguments and
 * results as gdn_quantized_matmul without workspace and workspace_bytes.
 * No counterpart in the reference (MLX's kernels allocate their own
 * scratch): for callers that cannot allocate device memory, such as code
 * under HIP graph capture, tight serving loops and harnesses that forbid
 * hipMalloc.
 */
int gdn_quantized_matmul_noalloc(const void *x, int x_dtype, const void *w, const void *scales,
                                 const void *biases, int sb_dtype, void *y, int y_dtype,
                                 const void *residual, int M, int N, int K, int bits, int group_size,
                                 void *stream);

/*
 * gdn_quantized_matmul_workspace_size - workspace bytes gdn_quantized_matmul
 * uses for these sizes and dtypes with its full K split (0: it does not
 * split K). No reference counterpart: MLX's kernels allocate their own.
 */
int64_t gdn_quantized_matmul_workspace_size(int x_dtype, int sb_dtype, int M, int N, int K,
                                            int bits, int group_size);

/* Quantization modes (the reference's QuantScheme.mode, config.py:17-33). */
#define GDN_QUANT_AFFINE 0
#define GDN_QUANT_MXFP4 1
#define GDN_QUANT_MXFP8 2
#define GDN_QUANT_NVFP4 3

/*
 * gdn_dequantize - the dense weights of a quantized projection, for every
 * scheme the reference's QuantScheme accepts. w: (N, K * bits / 32) uint32,
 * element k of row n the bits-wide field at bit bits * k of the row's
 * little-endian bit stream (for 2, 4 and 8 bits: bits [bits * (k % (32 /
 * bits)), +bits) of word k / (32 / bits)). out: (N, K) out_dtype.
 *   GDN_QUANT_AFFINE (bits 2, 3, 4, 5, 6 or 8; group_size 32, 64 or 128):
 *     out[n][k] = scales[n][g] * q + biases[n][g] (float32 product, one
 *     rounding to out_dtype), scales and biases (N, K / group_size) sb_dtype
 *   GDN_QUANT_MXFP4 (4 bits, group 32), GDN_QUANT_MXFP8 (8 bits, group 32),
 *   GDN_QUANT_NVFP4 (4 bits, group 16): the code's e2m1 (fp4) or e4m3 (fp8)
 *     value times its group's scale, (N, K / group_size) uint8: e8m0 (2^(s -
 *     127)) for the mx formats, e4m3 for nvfp4; biases unused (NULL); exact
 *     in float32 and bf16
 * Counterpart of mx.dequantize, which the reference's tests use to build dense
 * weights (tests/test_qwen3_5_linear_attention.py:59-70).
 */
int gdn_dequantize(const void *w, const void *scales, const void *biases, int sb_dtype, void *out,
                   int out_dtype, int N, int K, int bits, int group_size, int mode, void *stream);

/*
 * gdn_quantized_matmul_scheme - y = x W^T (+ residual) at decode sizes for
 * every scheme gdn_dequantize accepts (w, scales, biases, mode as there),
 * multiplied straight from the packed codes: the weight is read once at its
 * packed size and never expanded in memory. x: (M, K) bf16, 16-byte aligned,
 * M <= 64; y, residual: (M, N) y_dtype (residual may be NULL or equal y, as
 * in gdn_quantized_matmul). K a multiple of 32 and of group_size. float32
 * partial sums per 32-k block: affine adds s * sum(x q) + b * sum(x), the
 * float formats sum x times the exact product of code and scale. Where the
 * 64-column tiles are too few to fill the GPU, K is split over workgroups
 * whose float32 partial blocks (workspace, 16-byte aligned, at least
 * gdn_quantized_matmul_scheme_workspace_size bytes for the full split; a
 * smaller or NULL one splits less) are added in split order by a second
 * kernel. Returns GDN_EINVAL for sizes or schemes outside these.
 * Replaces mx.quantized_matmul(x, w, scales, biases, transpose=True,
 * group_size, bits, mode) at decode sizes (model/moe_block.py:44-55) for the
 * schemes gdn_quantized_matmul does not take (affine 2, 3, 5, 6 bits and the
 * float formats).
 */
int gdn_quantized_matmul_scheme(const void *x, const void *w, const void *scales, const void *biases,
                                int sb_dtype, void *y, int y_dtype, const void *residual, int M, int N,
                                int K, int bits, int group_size, int mode, void *workspace,
                                int64_t workspace_bytes, void *stream);

/* Workspace bytes gdn_quantized_matmul_scheme splits K with for these sizes
 * (0: no split). No reference counterpart: MLX's kernels allocate their own. */
int64_t gdn_quantized_matmul_scheme_workspace_size(int M, int N, int K);

#ifdef __cplusplus
}
#endif

#endif /* GDN_H */
