/*
 * fused_decode.h - C ABI of libfused_decode_hip.so, the gfx950 (MI355X) kernels
 * behind the Python package `fused_decode`.
 *
 * The reference has no C or FFI layer: its operators are Python functions in
 * src/fused_decode/ops.py that call Triton launchers in src/fused_decode/kernels.py.
 * Each entry point below replaces one of those launchers (cited per function) and
 * keeps the launcher's contract:
 *   - the caller owns every buffer; nothing here allocates device memory;
 *   - work is enqueued on the given stream (a hipStream_t passed as void*; NULL is
 *     the legacy default stream) and nothing synchronises, so a caller may capture
 *     the calls into a hipGraph;
 *   - inputs are read-only, except that residual_out may alias residual, and an
 *     output may alias the input it is computed from element-for-element (in-place
 *     norm, rope, swiglu);
 *   - arguments are checked before any HIP call: a bad argument returns
 *     FD_EINVAL and launches nothing. fd_last_error() gives the reason.
 *
 * Activations are float16 or bfloat16 (act_dtype), arithmetic is float32 with one
 * rounding per stored tensor. Strides and sizes are in elements, not bytes.
 */
#ifndef FUSED_DECODE_H
#define FUSED_DECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
enum { FD_F16 = 0, FD_BF16 = 1, FD_F32 = 2 };

/* GEMV kinds: the names of kernels.py:581-586 (`resolve_kind`). */
enum { FD_KIND_DOT = 0, FD_KIND_SIMT = 1 };

/* status codes */
enum {
  FD_OK = 0,
  FD_EINVAL = 1,      /* bad argument; nothing was launched */
  FD_EUNSUPPORTED = 2, /* valid, but outside what this build handles (e.g. LDS budget) */
  FD_ELAUNCH = 3      /* the HIP launch itself failed */
};

/*
 * A row layout: the tensor is a grid of a*b*c rows of n elements. Row (i,j,l)
 * starts at i*sa + j*sb + l*sc and element t of a row sits at t*col further on.
 * Any stride may be 0 (broadcast). Mirrors RowLayout of kernels.py:26-70.
 */
typedef struct fd_rows {
  int64_t a, b, c;
  int64_t sa, sb, sc;
  int64_t col;
  int64_t n;
} fd_rows;

/* Version of this library (major*10000 + minor*100 + patch). */
int fd_version(void);

/* HIP runtime version the library is bound to (hipRuntimeGetVersion). */
int fd_runtime_version(int* version);

/* Human-readable reason for the last non-OK status returned on this thread. */
const char* fd_last_error(void);

/*
 * Set-up, once per process, before any graph capture: resolves the library's
 * per-device state on every visible device (the device address of the no-alloc
 * entry point's array, which must not be looked up while a stream is being
 * captured). Makes each device current in turn and restores the caller's
 * device. FD_OK with no visible device; safe to call again (cheap). The Python
 * loaders call it when they load the library on a machine with a GPU.
 * No counterpart in the reference (its launchers need no set-up).
 */
int fd_init(void);

/*
 * y = x * rsqrt(mean(x^2) + eps) * w, per row, float32 reduction.
 * Replaces kernels.py:343-414 (`rms_out` without residual), launched from
 * ops.py:72-88 (`rms_norm`). w has n elements at stride w_stride, dtype w_dtype
 * (FD_F16, FD_BF16 or FD_F32).
 */
int fd_rms_norm(void* y, const void* x, const void* w, int w_dtype, int64_t w_stride,
                const fd_rows* lx, const fd_rows* ly, float eps, int act_dtype,
                void* stream);

/*
 * s = x + residual in float32; residual_out = round(s);
 * y = round(s * rsqrt(mean(s^2) + eps) * w) - the norm uses the float32 sum.
 * Replaces kernels.py:343-414 (`rms_out` with residual and residual_out),
 * launched from ops.py:91-119 (`add_rms_norm`). residual_out may alias residual.
 */
int fd_add_rms_norm(void* y, void* residual_out, const void* x, const void* residual,
                    const void* w, int w_dtype, int64_t w_stride, const fd_rows* lx,
                    const fd_rows* lr, const fd_rows* ly, const fd_rows* lro, float eps,
                    int act_dtype, void* stream);

/*
 * y = round(silu(gate) * up), float32 math with a stable sigmoid.
 * Replaces kernels.py:456-487 (`swiglu_out`), launched from ops.py:163-178.
 */
int fd_swiglu(void* y, const void* gate, const void* up, const fd_rows* lg,
              const fd_rows* lu, const fd_rows* ly, int act_dtype, void* stream);

/*
 * Rotate-half RoPE over rows of even length n, h = n/2:
 *   y[:h] = x1*c1 - x2*s1,  y[h:] = x2*c2 + x1*s2   (float32, one rounding).
 * cos/sin rows (dtype cs_dtype: FD_F16, FD_BF16 or FD_F32) use their own layouts,
 * typically with stride-0 broadcast dims.
 * Replaces kernels.py:541-578 (`rope_out`), launched from ops.py:138-160.
 */
int fd_rope(void* y, const void* x, const void* cos, const void* sin, int cs_dtype,
            const fd_rows* lx, const fd_rows* lc, const fd_rows* ls, const fd_rows* ly,
            int act_dtype, void* stream);

/*
 * y[m,n] = round(sum_k x[m,k] * w[n,k] + bias[n] + row_add[m,n]) for M <= 16.
 * w is [N,K] like F.linear. bias (optional, NULL for none) has dtype bias_dtype
 * (act_dtype or FD_F32) and stride sb; row_add (optional) has dtype row_dtype
 * (FD_F16/FD_BF16/FD_F32) and strides srm, srn (0 broadcasts). kind is
 * FD_KIND_DOT or FD_KIND_SIMT.
 * Replaces kernels.py:741-830 (`linear_out`, kernels `_linear_dot` :606-672 and
 * `_linear_simt` :675-738), launched from ops.py:212-280 (`linear_decode`).
 */
int fd_linear(void* y, const void* x, const void* w, const void* bias, int bias_dtype,
              const void* row_add, int row_dtype, int64_t M, int64_t N, int64_t K,
              int64_t sxm, int64_t sxk, int64_t swn, int64_t swk, int64_t sb,
              int64_t srm, int64_t srn, int64_t sym, int64_t syn, int kind, int act_dtype,
              void* stream);

/*
 * GEMV tiling: weight rows per workgroup, which also names the kernel (2, 4 or 8:
 * the SIMT kernel, 8 only up to M = 8; 16: the MFMA kernel, kind FD_KIND_DOT
 * only), waves per workgroup (SIMT 1..8; MFMA 2, 4 or 8) and stages: for the
 * MFMA kernel, K units of 128 each wave keeps in flight in its LDS ring (1..3; 2
 * by default; waves x units must fit one CU's LDS); for the SIMT kernel its form
 * (0 the library's choice, 1 one workgroup per tile, 2 the persistent kernel that
 * keeps the activations in registers, whose waves then set how many 512-element
 * K chunks each lane holds). 0 = the library's default for that field; with rows
 * 0 the kernel is chosen as in fd_linear (MFMA for kind FD_KIND_DOT from M = 5).
 */
typedef struct fd_tile {
  int rows;
  int waves;
  int stages;
} fd_tile;

/*
 * fd_linear with an explicit tiling (`tile` may be NULL: the defaults). A tile
 * the running kernel does not accept is FD_EINVAL. Replaces the tile override of
 * kernels.py:589-603 (`linear_config` reading FUSED_DECODE_LINEAR), which the
 * Python layer maps onto this call, and serves the tile search that replaces
 * bench.py:475-517 (`tune`).
 */
int fd_linear_tiled(void* y, const void* x, const void* w, const void* bias, int bias_dtype,
                    const void* row_add, int row_dtype, int64_t M, int64_t N, int64_t K,
                    int64_t sxm, int64_t sxk, int64_t swn, int64_t swk, int64_t sb,
                    int64_t srm, int64_t srn, int64_t sym, int64_t syn, const fd_tile* tile,
                    int kind, int act_dtype, void* stream);

/*
 * Llama post-attention MLP for a contiguous hidden [M,H], M <= 16:
 *   h   = round(rms_norm(hidden, norm_w, eps))
 *   g,u = round(h @ w_gate_up[:I].T), round(h @ w_gate_up[I:].T)
 *   mid = round(silu(g) * u)                      (written to `mid`, [M,I])
 *   y   = round(mid @ w_down.T + hidden)
 * w_gate_up is [2I,H] (gate rows above up rows), w_down is [H,I], both contiguous.
 * `mid` is caller-owned scratch of M*I activation elements. y, mid and hidden must
 * not share memory (FD_EINVAL): hidden is read as the residual after y and mid are
 * written. Two launches (three for kind FD_KIND_DOT at M >= 9, whose RMSNorm runs
 * as its own row kernel into y; from 5 to 8 rows the MFMA gate/up kernel
 * normalises hidden itself, for H up to about 35,000).
 * Replaces the composition at ops.py:283-315 (`post_attn_mlp`), which runs four
 * launches (rms_norm, linear_decode, swiglu, linear_decode with row_add).
 */
int fd_post_attn_mlp(void* y, void* mid, const void* hidden, const void* norm_w,
                     int norm_w_dtype, const void* w_gate_up, const void* w_down,
                     int64_t M, int64_t H, int64_t I, float eps, int kind, int act_dtype,
                     void* stream);

/*
 * fd_post_attn_mlp without the `mid` argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. `mid` lives in a
 * library-owned device array of 1 MiB per GPU (held until the process ends):
 * M*I*2 must not exceed 1,048,576 bytes (FD_EINVAL otherwise; Llama-3-8B widths
 * at M = 16 need 458,752). The call allocates nothing and runs the same kernels,
 * with the same results, as fd_post_attn_mlp. Every call on one GPU shares that
 * GPU's array: calls that may overlap on one GPU (different streams, or host
 * threads) race and must be serialised by the caller. Nothing in the array needs
 * to start at zero (the gate/up launch writes all M*I values before the down
 * projection reads them). The array's address is resolved per device by fd_init;
 * a caller that skipped fd_init gets it looked up on its first call on each
 * device (the stream's device), which must then not be under graph capture.
 */
int fd_post_attn_mlp_noalloc(void* y, const void* hidden, const void* norm_w, int norm_w_dtype,
                             const void* w_gate_up, const void* w_down, int64_t M, int64_t H,
                             int64_t I, float eps, int kind, int act_dtype, void* stream);

/*
 * The gate/up half of fd_post_attn_mlp alone: mid = round(silu(round(g)) * round(u))
 * with g,u = round(round(rms_norm(hidden)) @ w_gate_up.T) split at I. Same operand
 * rules as fd_post_attn_mlp. With kind FD_KIND_DOT and M >= 9 (or H above about
 * 35,000 from M = 5) the RMSNorm is
 * written to `normed` ([M,H] activation scratch, 16-byte aligned) by a row kernel
 * before the MFMA gate/up kernel reads it; otherwise `normed` is unused (may be
 * NULL) and a single kernel normalises in its prologue. For callers that run their
 * own down projection, and for timing the dominant kernel of the block on its own.
 * Replaces ops.py:312-314 (rms_norm, the gate/up linear_decode and swiglu).
 */
int fd_mlp_gate_up(void* mid, void* normed, const void* hidden, const void* norm_w,
                   int norm_w_dtype, const void* w_gate_up, int64_t M, int64_t H, int64_t I,
                   float eps, int kind, int act_dtype, void* stream);

/*
 * Pre-attention QKV projection of a decode step in one launch:
 *   h   = round(rms_norm(hidden, norm_w, eps))                       [M,H]
 *   qkv = round(h @ w_qkv.T + bias)                                  [M,N]
 *   y   = qkv with rope(qkv[:, :rope_cols] viewed as heads of head_dim, cos, sin)
 * rope is the rotate-half of fd_rope, applied to the rounded projection; cos/sin
 * row m (head_dim values of cs_dtype, unit stride) sits at m * cs_row_stride, and
 * cs_row_stride 0 shares one row across all M. hidden [M,H], w_qkv [N,H] and y
 * [M,N] are contiguous; bias ([N], bias_dtype) may be NULL. rope_cols is a
 * multiple of head_dim (0: no rotation); this build needs head_dim % 16 == 0 and
 * H % 8 == 0 (FD_EUNSUPPORTED otherwise: compose fd_rms_norm, fd_linear, fd_rope).
 * With kind FD_KIND_DOT from M = 7 the projection runs on MFMA with the RMSNorm
 * folded into the kernel (any H when norm_w has act_dtype, which streams with
 * the weights; another norm_w dtype is staged in LDS as float32, which takes H
 * up to about 22,000, FD_EUNSUPPORTED beyond); below that, or with
 * FD_KIND_SIMT, a SIMT kernel normalises in its prologue (up to 8 rows the
 * persistent one, which holds the normalised rows in registers, where H fits
 * eight waves of up to four 512-element chunks per lane). `normed` is unused at
 * every M and may be NULL (it stays in the signature for callers written against
 * earlier builds).
 * No reference counterpart as one call: it fuses the composition a caller of the
 * reference writes from rms_norm (ops.py:72-88), linear_decode (ops.py:212-280)
 * and rope (ops.py:138-160) on the q and k heads, the first cross-op fusion the
 * decode step names after the MLP block.
 */
int fd_pre_attn_qkv(void* y, void* normed, const void* hidden, const void* norm_w,
                    int norm_w_dtype, const void* w_qkv, const void* bias, int bias_dtype,
                    const void* cos, const void* sin, int cs_dtype, int64_t cs_row_stride,
                    int64_t M, int64_t H, int64_t N, int64_t rope_cols, int64_t head_dim,
                    float eps, int kind, int act_dtype, void* stream);

/*
 * GEMV with FP8 weights (OCP E4M3, one byte per weight, row stride swn in bytes)
 * and one float32 scale per output row:
 *   y[m,n] = round(w_scale[n] * sum_k e4m3(w8[n,k]) * x[m,k] + bias[n] + row_add[m,n])
 * M <= 16; x [M,K] activations with unit K stride; K % 16 == 0 and 16-byte
 * aligned rows (else FD_EUNSUPPORTED). bias/row_add as in fd_linear. The
 * weights are decoded exactly (codes 0x7f and 0xff are NaN, as torch's
 * float8_e4m3fn has them) and the arithmetic is float32: the activations are
 * never quantised.
 * No reference counterpart (its weights are fp16/bf16 only): a low-precision
 * weight format, halving the bytes the decode GEMV streams.
 */
int fd_linear_fp8(void* y, const void* x, const void* w8, const float* w_scale,
                  const void* bias, int bias_dtype, const void* row_add, int row_dtype,
                  int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t swn, int64_t sb,
                  int64_t srm, int64_t srn, int64_t sym, int64_t syn, int act_dtype,
                  void* stream);

/*
 * fd_post_attn_mlp with FP8 weights: w_gate_up8 [2I,H] and w_down8 [H,I] E4M3
 * codes (contiguous) with per-row float32 scales gate_up_scale [2I] and
 * down_scale [H]; each projection is fd_linear_fp8's product, with the same four
 * rounding points as fd_post_attn_mlp. Two launches at every M (fused RMSNorm +
 * gate/up + SwiGLU, from M = 5 on MFMA with the norm weight staged in LDS, which
 * takes H up to about 38,000: FD_EUNSUPPORTED beyond; at 5-8 rows with H a
 * multiple of 512 and a float32 or activation-type norm weight the persistent
 * MFMA form, one workgroup per CU with the normalised rows resident in LDS; at
 * 2-4 rows the persistent SIMT kernel; then down + residual);
 * `mid` is caller scratch of M*I activations. y, mid and hidden must not share
 * memory (FD_EINVAL). H % 16 == 0 and I % 16 == 0. No reference counterpart (see
 * fd_linear_fp8).
 */
int fd_post_attn_mlp_fp8(void* y, void* mid, const void* hidden, const void* norm_w,
                         int norm_w_dtype, const void* w_gate_up8, const float* gate_up_scale,
                         const void* w_down8, const float* down_scale, int64_t M, int64_t H,
                         int64_t I, float eps, int act_dtype, void* stream);

/*
 * fd_pre_attn_qkv with FP8 weights: w_qkv8 [N,H] E4M3 codes (contiguous) with
 * per-row float32 scales w_scale [N]; the projection is fd_linear_fp8's product
 * and everything else (RMSNorm, bias, rounding, RoPE of the first rope_cols
 * columns, cos/sin layout) is fd_pre_attn_qkv's. One launch at every M (at 2-4
 * rows the persistent SIMT kernel, from M = 5 the MFMA form, each with the
 * RMSNorm folded in); `normed` is unused and may
 * be NULL (kept for the fp16 entry point's signature). H % 16 == 0 and
 * head_dim % 16 == 0 (else FD_EUNSUPPORTED). No reference counterpart (see
 * fd_linear_fp8 and fd_pre_attn_qkv).
 */
int fd_pre_attn_qkv_fp8(void* y, void* normed, const void* hidden, const void* norm_w,
                        int norm_w_dtype, const void* w_qkv8, const float* w_scale,
                        const void* bias, int bias_dtype, const void* cos, const void* sin,
                        int cs_dtype, int64_t cs_row_stride, int64_t M, int64_t H, int64_t N,
                        int64_t rope_cols, int64_t head_dim, float eps, int act_dtype,
                        void* stream);

/*
 * Row sums of squares handed from a producer launch to the next RMSNorm
 * (decode-step chaining; the MFMA kernels only: kind FD_KIND_DOT, or the fp8
 * forms, with 5 <= M <= 16, else FD_EUNSUPPORTED). A producer that writes an
 * [M,N] activation also writes `ss_out`: ceil(N/16) tiles of 16 floats,
 * ss_out[t*16 + m] = sum over the tile's columns n of round(y[m,n])^2 in float32
 * (0 for m >= M). A consumer whose RMSNorm input is that activation (width H)
 * takes `ss_in` (ss_tiles = ceil(H/16), else FD_EINVAL) and derives
 * rsqrt(mean(x^2) + eps) from it instead of re-reading the rows: the MLP's
 * RMSNorm then runs inside the gate/up kernel (no row kernel), the QKV kernel
 * skips its pass over x. Results are the operators' (the same float32 sum of
 * squares, added in another order). ss_in must hold the sums of exactly the
 * `hidden` passed with it; ss_in/ss_out are 16-byte aligned (FD_EUNSUPPORTED).
 * No reference counterpart: the reference's operators each normalise their own
 * input (ops.py:72-88, composed at ops.py:312-315).
 *
 * fd_linear_sumsq: fd_linear plus ss_out (non-NULL).
 * fd_post_attn_mlp_sumsq: fd_post_attn_mlp; ss_in may be NULL (the MLP then
 *   normalises as in fd_post_attn_mlp), ss_out may be NULL.
 * fd_pre_attn_qkv_sumsq: fd_pre_attn_qkv without `normed`, ss_in non-NULL (at 5-6
 *   rows the persistent SIMT QKV runs, which sums the squares of the rows it holds
 *   in registers anyway and does not read ss_in).
 * The _fp8 forms are the same over fd_linear_fp8, fd_post_attn_mlp_fp8 and
 * fd_pre_attn_qkv_fp8.
 */
int fd_linear_sumsq(void* y, const void* x, const void* w, const void* bias, int bias_dtype,
                    const void* row_add, int row_dtype, int64_t M, int64_t N, int64_t K,
                    int64_t sxm, int64_t sxk, int64_t swn, int64_t swk, int64_t sb, int64_t srm,
                    int64_t srn, int64_t sym, int64_t syn, int kind, int act_dtype, float* ss_out,
                    void* stream);
int fd_post_attn_mlp_sumsq(void* y, void* mid, const void* hidden, const void* norm_w,
                           int norm_w_dtype, const void* w_gate_up, const void* w_down, int64_t M,
                           int64_t H, int64_t I, float eps, int kind, int act_dtype,
                           const float* ss_in, int64_t ss_tiles, float* ss_out, void* stream);
int fd_pre_attn_qkv_sumsq(void* y, const void* hidden, const void* norm_w, int norm_w_dtype,
                          const void* w_qkv, const void* bias, int bias_dtype, const void* cos,
                          const void* sin, int cs_dtype, int64_t cs_row_stride, int64_t M,
                          int64_t H, int64_t N, int64_t rope_cols, int64_t head_dim, float eps,
                          int kind, int act_dtype, const float* ss_in, int64_t ss_tiles,
                          void* stream);
int fd_linear_fp8_sumsq(void* y, const void* x, const void* w8, const float* w_scale,
                        const void* bias, int bias_dtype, const void* row_add, int row_dtype,
                        int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t swn, int64_t sb,
                        int64_t srm, int64_t srn, int64_t sym, int64_t syn, int act_dtype,
                        float* ss_out, void* stream);
int fd_post_attn_mlp_fp8_sumsq(void* y, void* mid, const void* hidden, const void* norm_w,
                               int norm_w_dtype, const void* w_gate_up8,
                               const float* gate_up_scale, const void* w_down8,
                               const float* down_scale, int64_t M, int64_t H, int64_t I,
                               float eps, int act_dtype, const float* ss_in, int64_t ss_tiles,
                               float* ss_out, void* stream);
int fd_pre_attn_qkv_fp8_sumsq(void* y, const void* hidden, const void* norm_w, int norm_w_dtype,
                              const void* w_qkv8, const float* w_scale, const void* bias,
                              int bias_dtype, const void* cos, const void* sin, int cs_dtype,
                              int64_t cs_row_stride, int64_t M, int64_t H, int64_t N,
                              int64_t rope_cols, int64_t head_dim, float eps, int act_dtype,
                              const float* ss_in, int64_t ss_tiles, void* stream);

/*
 * Bandwidth roofs. dst = src over `bytes` bytes (any size; 16-byte aligned
 * pointers take the vector path). c = a + b*scale over n elements of dtype.
 * Replace kernels.py:833-858 (`launch_copy`, `launch_triad`).
 */
int fd_copy(void* dst, const void* src, int64_t bytes, void* stream);
int fd_triad(void* c, const void* a, const void* b, float scale, int64_t n, int dtype,
             void* stream);

/*
 * Read roof: streams `bytes` bytes from src (16-byte aligned, bytes % 16 == 0,
 * else FD_EUNSUPPORTED) with the copy's load pattern and stores nothing but a
 * flag: *hit (a device word, 4-byte aligned) gets bit 0 set where the xor of
 * the words one wave read equals `key`, so the loads cannot be elided. The
 * ceiling of a kernel that only streams, as the decode GEMVs do. No reference
 * counterpart (its bench has the copy and the triad).
 */
int fd_read(const void* src, int64_t bytes, int key, void* hit, void* stream);

/*
 * The copy roof's persistent form: dst = src over `bytes` bytes with a fixed
 * grid of `workgroups` 256-thread workgroups walking the 16-byte vectors
 * grid-stride, four per thread per pass (16-byte aligned pointers and bytes %
 * 16 == 0, else FD_EUNSUPPORTED). On copies of tens of MB it can beat fd_copy's
 * one-pass grid, so the bench times both and takes the faster as a kernel's
 * same-size copy ceiling. No reference counterpart.
 */
int fd_copy_persistent(void* dst, const void* src, int64_t bytes, int workgroups, void* stream);

/*
 * Clock probe, a measurement aid: `workgroups` (1..4096) one-wave workgroups
 * each write three uint64 to out[3*i..3*i+2] (8-byte aligned): where it ran
 * (XCD id << 8 | the SE, SH and CU fields of HW_ID), that CU's shader clock
 * counter (s_memtime) and the constant-rate wall clock (s_memrealtime), whose
 * rate in kHz goes to *wall_khz. The shader counters of different CUs are not
 * synchronised: probes before and after a piece of work on one stream are
 * compared CU by CU, each CU's counter advance over the wall clock's being
 * proportional to its gfx clock during the work. No reference counterpart.
 */
int fd_clock_probe(unsigned long long* out, int workgroups, int* wall_khz, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FUSED_DECODE_H */
