// GEMV and fused post-attention MLP with FP8 (OCP E4M3) weights for gfx950.
//
//   y[m,n] = round(scale[n] * sum_k e4m3(w[n,k]) * x[m,k] + bias[n] + row_add[m,n])
//
// Weights are one byte each with one float32 scale per output row (per-channel
// quantisation), so a decode GEMV streams half the bytes of the fp16 one. The
// activations stay fp16/bf16 and the arithmetic float32: weights are decoded
// exactly, never the activations quantised.
//
// Decode: gfx950's v_cvt_scalef32_pk_f16_fp8 / _bf16_fp8 (scale 1) turn two
// codes into a pair of the activation type; every E4M3 value (NaN included) is
// exact in fp16 and in bf16, so four codes cost two conversions and the
// products are those of the exact weights. v_dot2 then takes two products per
// op into float32.
//
// Layout per SIMT step (M < 5): a lane streams 16 consecutive codes (16 bytes) of
// each of its workgroup's R rows, so a wave covers 1024 K elements per step.
// From 5 rows the products run on MFMA: the GEMV and the fused QKV in the DMA
// GEMV of fd_dma.h (codes decoded after their LDS read), the MLP's gate/up in a
// relayout kernel that decodes the codes into an LDS tile.

#include <type_traits>

#include "fd_dma.h"
#include "fd_gemv.h"
#include "fd_res.h"
#include "fd_internal.h"

namespace fd {

constexpr int kChunk8 = 1024;  // K elements one wave covers per fp8 step

// Four E4M3 codes (byte 0 first) -> two pairs of their exact values in T.
template <typename T>
__device__ __forceinline__ void fp8x4_to_pairs(uint32_t w, uint32_t& lo, uint32_t& hi);
template <>
__device__ __forceinline__ void fp8x4_to_pairs<f16>(uint32_t w, uint32_t& lo, uint32_t& hi) {
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
  hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
}
template <>
__device__ __forceinline__ void fp8x4_to_pairs<bf16>(uint32_t w, uint32_t& lo, uint32_t& hi) {
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
  hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc, f16) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
}
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc, bf16) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b),
                                         acc, false);
}

// acc += sum over 16 elements of e4m3(weight) * x, x given as two 8-element
// vectors (elements 0-7, 8-15).
template <typename T>
__device__ __forceinline__ float dot_fp8x16(const u32x4& w, const typename Vec8<T>::type& xa,
                                            const typename Vec8<T>::type& xb, float acc) {
  const u32x4 xa2 = __builtin_bit_cast(u32x4, xa), xb2 = __builtin_bit_cast(u32x4, xb);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t lo, hi;
    fp8x4_to_pairs<T>(w[i], lo, hi);
    const uint32_t x0 = i < 2 ? xa2[2 * i] : xb2[2 * i - 4];
    const uint32_t x1 = i < 2 ? xa2[2 * i + 1] : xb2[2 * i - 3];
    acc = dot2(lo, x0, acc, T{});
    acc = dot2(hi, x1, acc, T{});
  }
  return acc;
}

__device__ __forceinline__ u32x4 load16_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// SIMT fp8 GEMV: R rows per workgroup, waves split K in 1024-element chunks,
// transposing butterfly + LDS across waves, then scale, bias, row_add, rounding.
// A wave's K steps run through stream_steps with every load unconditional (a
// lane past K reads chunk 0, masked in the math), so each wave has its next
// step's codes and activations in flight while it multiplies the current one.
template <typename T, int M, int R>
struct Step8Regs {
  u32x4 w[R];
  typename Vec8<T>::type xa[M], xb[M];
};

template <typename T, int M, int R>
__global__ __launch_bounds__(kMaxWaves * kWave) void gemv_fp8_kernel(
    T* y, const T* x, const uint8_t* w, const float* wscale, int N, int K, int64_t sxm,
    int64_t swn, int64_t sym, int64_t syn, Epi e) {
  constexpr int V = pow2_ceil(R * M);
  __shared__ float part[kMaxWaves * V];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = block_threads() / kWave;
  const int64_t n0 = (int64_t)blockIdx.x * R;
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  const uint8_t* wr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wr[r] = w + (n0 + r < N ? n0 + r : 0) * swn;  // rows past N: never stored
  const int step = nw * kChunk8;
  const int steps = (K + step - 1) / step;
  const int kbase = (wave * kWave + lane) * 16;
  auto issue = [&](Step8Regs<T, M, R>& q, int s) {
    const int k = kbase + s * step;
    const int kc = k < K ? k : 0;
#pragma unroll
    for (int r = 0; r < R; ++r) q.w[r] = load16_nt(wr[r] + kc);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      q.xa[m] = load8<T>(x + m * sxm + kc);
      q.xb[m] = load8<T>(x + m * sxm + kc + 8);
    }
  };
  auto consume = [&](const Step8Regs<T, M, R>& q, int s) {
    if (kbase + s * step >= K) return;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r * M + m] = dot_fp8x16<T>(q.w[r], q.xa[m], q.xb[m], acc[r * M + m]);
  };
  Step8Regs<T, M, R> qa, qb;
  if (steps > 0) issue(qa, 0);  // K = 0 loads nothing (x may be null)
  stream_steps(steps, qa, qb, issue, consume);
  butterfly_sum<V>(acc, lane);
  if (butterfly_writer<V>(lane)) part[wave * V + butterfly_index<V>(lane)] = acc[0];
  __syncthreads();
  for (int t = threadIdx.x; t < R * M; t += block_threads()) {
    const int r = t / M, m = t % M;
    const int64_t n = n0 + r;
    if (n < N) {
      float s = 0.f;
      for (int i = 0; i < nw; ++i) s += part[i * V + t];
      y[m * sym + n * syn] = from_f32<T>(epilogue(e, s * wscale[n], m, n));
    }
  }
}

// v_dot2 of a pair with a pair and an inline-constant zero addend (the first
// product of a sum: no register is zeroed first).
__device__ __forceinline__ float dot2_first(uint32_t a, uint32_t b, f16) {
  float r;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float dot2_first(uint32_t a, uint32_t b, bf16) {
  float r;
  asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// Persistent SIMT GEMV with E4M3 weights, the layout of gemv_simt_px_kernel
// with one 16-byte load of 16 codes per lane, row and chunk: each wave keeps
// its CPL 1024-element K chunks of the M activation rows in registers (8 pairs
// per row and chunk), and the workgroup walks every gridDim-th tile of R rows,
// decoding each lane's codes exactly to T pairs once per row before the M
// rows' v_dot2s. After the last tile it adds the waves' sums and applies the
// channel scale and the epilogue. kPxQkv: the RMSNorm is applied to the
// registers first (as qkv_px_kernel), the rows are placed by TileRows<R>, and
// the epilogue scales, adds the bias, rounds and rotates (y is [M, N]).
// kPxGateUp: the same RMSNorm; a tile is R/2 gate rows j.. and the matching up
// rows I + j.. of w [2I, K] (N = 2I), and the epilogue writes
// y[m, j] = round(silu(round(g * s_g)) * round(u * s_u)) into y [M, I].
enum Fp8PxMode { kPxGemv = 0, kPxQkv = 1, kPxGateUp = 2 };
template <typename T, int M, int R, int CPL, int MODE>
__global__ __launch_bounds__(kMaxWaves * kWave) void fp8_px_kernel(
    T* y, const T* x, const uint8_t* w, const float* wscale, int N, int K, int64_t sxm, int64_t swn,
    int64_t sym, int64_t syn, Epi e, int tiles, const void* nwp, int nw_dtype, float eps, Rope rp) {
  constexpr int V = pow2_ceil(R * M);
  constexpr int MP = pow2_ceil(M);
  constexpr int P = R / 2;  // kPxQkv: pairs per rotated tile; kPxGateUp: gate rows per tile
  const int I = N / 2;       // kPxGateUp: the gate (and up) rows
  extern __shared__ __align__(16) float pxs8[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int nt = block_threads(), nw = nt / kWave;
  const int g = (int)gridDim.x;
  const int mine = ((int)blockIdx.x < tiles) ? (tiles - (int)blockIdx.x + g - 1) / g : 0;
  float* parts = pxs8;                        // [my tile][wave][V]
  float* ssq = pxs8 + (size_t)mine * nw * V;  // norm: [wave][MP], then inv[MP]
  float* inv = ssq + kMaxWaves * MP;
  int kc[CPL];
  bool kin[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int k = ((wave + c * nw) * kWave + lane) * 16;
    kin[c] = k < K;
    kc[c] = kin[c] ? k : 0;
  }
  const bool whole = ((wave + (CPL - 1) * nw) * kWave + kWave - 1) * 16 < K;
  auto row_of = [&](int i, int r) -> int64_t {
    const int tile = (int)blockIdx.x + i * g;
    if constexpr (MODE == kPxQkv) {
      return TileRows<R>(rp, tile).row(r);
    } else if constexpr (MODE == kPxGateUp) {
      const int64_t j = (int64_t)tile * P + (r % P);
      return r < P ? j : I + j;  // rows past I: loaded, never stored
    } else {
      return (int64_t)tile * R + r;
    }
  };
  struct Regs {
    u32x4 v[CPL][R];
  };
  auto issue = [&](Regs& q, int i) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = row_of(i, r);
      const uint8_t* wr = n < N ? w + n * swn : w;  // a wave-uniform row base
#pragma unroll
      for (int c = 0; c < CPL; ++c) q.v[c][r] = load16_nt(wr + kc[c]);
    }
  };
  // the activation rows (and the norm weight) first, then the first tile
  uint32_t xp[CPL][M][8];
  float wf[MODE != kPxGemv ? CPL : 1][16];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const u32x4 a = __builtin_bit_cast(u32x4, load8<T>(x + m * sxm + kc[c]));
      const u32x4 b = __builtin_bit_cast(u32x4, load8<T>(x + m * sxm + kc[c] + 8));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xp[c][m][j] = a[j];
        xp[c][m][j + 4] = b[j];
      }
    }
    if constexpr (MODE != kPxGemv) {
      float lo[8], hi[8];
      load8_norm_w(nwp, nw_dtype, kc[c], lo);
      load8_norm_w(nwp, nw_dtype, kc[c] + 8, hi);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        wf[c][j] = lo[j];
        wf[c][j + 8] = hi[j];
      }
    }
  }
  Regs a, b;
  if (mine > 0) issue(a, 0);
  if constexpr (MODE != kPxGemv) {
    float ss[MP];
#pragma unroll
    for (int m = 0; m < MP; ++m) ss[m] = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      if (kin[c]) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int j = 0; j < 8; ++j) ss[m] = sq_dot2<T>(xp[c][m][j], ss[m]);
      }
    butterfly_sum<MP>(ss, lane);
    if (butterfly_writer<MP>(lane)) ssq[wave * MP + butterfly_index<MP>(lane)] = ss[0];
    __syncthreads();
    if (tid < M) {
      float sum = 0.f;
      for (int i = 0; i < nw; ++i) sum += ssq[i * MP + tid];
      inv[tid] = rsqrtf(sum / (float)K + eps);
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CPL; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4 w0 = __builtin_bit_cast(u32x4, f32x4{wf[c][8 * h], wf[c][8 * h + 1], wf[c][8 * h + 2],
                                                         wf[c][8 * h + 3]});
        const u32x4 w1 = __builtin_bit_cast(u32x4, f32x4{wf[c][8 * h + 4], wf[c][8 * h + 5],
                                                         wf[c][8 * h + 6], wf[c][8 * h + 7]});
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const u32x4 raw{xp[c][m][4 * h], xp[c][m][4 * h + 1], xp[c][m][4 * h + 2], xp[c][m][4 * h + 3]};
          const u32x4 o = norm_frag<T>(raw, inv[m], w0, w1);
#pragma unroll
          for (int j = 0; j < 4; ++j) xp[c][m][4 * h + j] = o[j];
        }
      }
  }
  auto consume = [&](const Regs& q, int i) {
    float acc[V];
#pragma unroll
    for (int j = R * M; j < V; ++j) acc[j] = 0.f;
    if (whole) {
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          uint32_t pw[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) fp8x4_to_pairs<T>(q.v[c][r][j], pw[2 * j], pw[2 * j + 1]);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            float s = c == 0 ? dot2_first(pw[0], xp[c][m][0], T{}) : dot2(pw[0], xp[c][m][0], acc[r * M + m], T{});
#pragma unroll
            for (int j = 1; j < 8; ++j) s = dot2(pw[j], xp[c][m][j], s, T{});
            acc[r * M + m] = s;
          }
        }
    } else {
#pragma unroll
      for (int j = 0; j < R * M; ++j) acc[j] = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c)
        if (kin[c]) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            uint32_t pw[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) fp8x4_to_pairs<T>(q.v[c][r][j], pw[2 * j], pw[2 * j + 1]);
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
              for (int j = 0; j < 8; ++j) acc[r * M + m] = dot2(pw[j], xp[c][m][j], acc[r * M + m], T{});
          }
        }
    }
    butterfly_sum<V>(acc, lane);
    if (butterfly_writer<V>(lane)) parts[(i * nw + wave) * V + butterfly_index<V>(lane)] = acc[0];
  };
  stream_steps(mine, a, b, issue, consume);
  __syncthreads();
  if constexpr (MODE == kPxGateUp) {
    for (int t = tid; t < mine * P * M; t += nt) {
      const int i = t / (P * M), rm = t % (P * M);
      const float* pt = parts + (size_t)i * nw * V;
      const int r = rm / M, m = rm % M;
      const int64_t j = (int64_t)((int)blockIdx.x + i * g) * P + r;
      if (j < I) {
        float gs = 0.f, us = 0.f;
        for (int q = 0; q < nw; ++q) {
          gs += pt[q * V + rm];
          us += pt[q * V + P * M + rm];
        }
        y[m * (int64_t)I + j] = swiglu_out<T>(gs * wscale[j], us * wscale[I + j]);
      }
    }
    return;
  }
  for (int t = tid; t < mine * R * M; t += nt) {
    const int i = t / (R * M), rm = t % (R * M);
    const float* pt = parts + (size_t)i * nw * V;
    if constexpr (MODE == kPxQkv) {
      const TileRows<R> tr(rp, (int)blockIdx.x + i * g);
      if (tr.rotated()) {
        if (rm >= P * M) continue;  // one item per rotate-half pair
        const int p = rm / M, m = rm % M;
        float s1 = 0.f, s2 = 0.f;
        for (int j = 0; j < nw; ++j) {
          s1 += pt[j * V + p * M + m];
          s2 += pt[j * V + (p + P) * M + m];
        }
        const int64_t n1 = tr.row(p), n2 = tr.row(p + P);
        float o1, o2;
        rope_pair(rp, m, tr.col(p), round_as<T>(epilogue(e, s1 * wscale[n1], m, n1)),
                  round_as<T>(epilogue(e, s2 * wscale[n2], m, n2)), o1, o2);
        y[m * (int64_t)N + n1] = from_f32<T>(o1);
        y[m * (int64_t)N + n2] = from_f32<T>(o2);
        continue;
      }
    }
    const int r = rm / M, m = rm % M;
    const int64_t n = row_of(i, r);
    if (n < N) {
      float sum = 0.f;
      for (int j = 0; j < nw; ++j) sum += pt[j * V + rm];
      if constexpr (MODE == kPxQkv)
        y[m * (int64_t)N + n] = from_f32<T>(epilogue(e, sum * wscale[n], m, n));
      else
        y[m * sym + n * syn] = from_f32<T>(epilogue(e, sum * wscale[n], m, n));
    }
  }
}

// Fused gate/up + SwiGLU with fp8 weights: the RMSNorm prologue of the fp16
// kernel (normalised rows rounded into LDS), R gate rows and the matching R up
// rows per tile streamed through the step pipeline, and
// mid = round(silu(round(sg*g)) * round(su*u)).
template <int R>
struct GateUp8Regs {
  u32x4 g[R], u[R];
};

// Loads of step s of the plan; lanes past H and rows past I load the first 16
// codes instead (never used), so every load is unconditional.
template <int R>
__device__ __forceinline__ void load_gate_up8(GateUp8Regs<R>& b, const uint8_t* wgu,
                                              const StepPlan& p, int s, int H, int I) {
  const int64_t j0 = (int64_t)p.tile(s) * R;
  const int k = p.k(s);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t j = j0 + r;
    const bool ok = j < I && k < H;
    b.g[r] = load16_nt(ok ? wgu + j * H + k : wgu);
    b.u[r] = load16_nt(ok ? wgu + (I + j) * H + k : wgu);
  }
}

template <typename T, int M, int R, bool REGS>
__global__ __launch_bounds__(kMaxWaves * kWave) void mlp_gate_up_fp8_kernel(
    T* __restrict__ mid, const T* hidden, const void* nwp, int nw_dtype, const uint8_t* wgu,
    const float* __restrict__ gu_scale, int H, int I, float eps, int tiles) {
  typedef typename Vec8<T>::type V8;
  constexpr int V = pow2_ceil(2 * R * M);
  extern __shared__ __align__(16) unsigned char smem[];
  const int XS = xs_stride(H);
  T* xs = reinterpret_cast<T*>(smem);
  float* part = reinterpret_cast<float*>(smem + (size_t)M * XS * sizeof(T));
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = block_threads() / kWave;
  const StepPlan p(tiles, H, nw * kChunk8, (wave * kWave + lane) * 16);

  NormRegs<T, M, kNormRegRows(M)> nr;
  if constexpr (REGS) norm_load(nr, hidden, nwp, nw_dtype, M, H);
  GateUp8Regs<R> a, b;
  load_gate_up8<R>(a, wgu, p, 0, H, I);
  if constexpr (REGS)
    norm_store(nr, xs, part, nw_dtype, M, H, eps);
  else
    stage_normed<T, M>(xs, part, hidden, nwp, nw_dtype, M, H, eps);

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  auto issue = [&](GateUp8Regs<R>& buf, int s) { load_gate_up8<R>(buf, wgu, p, s, H, I); };
  auto consume = [&](const GateUp8Regs<R>& buf, int s) {
    const int k = p.k(s);
    if (k < H) {
      V8 xa[M], xb[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        xa[m] = load8<T>(xs + m * XS + k);
        xb[m] = load8<T>(xs + m * XS + k + 8);
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) {
          acc[r * M + m] = dot_fp8x16<T>(buf.g[r], xa[m], xb[m], acc[r * M + m]);
          acc[R * M + r * M + m] = dot_fp8x16<T>(buf.u[r], xa[m], xb[m], acc[R * M + r * M + m]);
        }
    }
    if (!p.last(s)) return;
    // The tile's channel scales sit at wave-uniform addresses: scalar loads,
    // which leave the next step's weight loads in flight (a vector load here
    // would be waited for behind them).
    const int j0 = p.tile(s) * R;
    float sg[R], su[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = __builtin_amdgcn_readfirstlane(j0 + r < I ? j0 + r : I - 1);
      sg[r] = gu_scale[j];
      su[r] = gu_scale[I + j];
    }
    butterfly_sum<V>(acc, lane);
    // Consecutive tiles alternate halves of `part`, so one barrier suffices: the
    // half written here was last read two tiles ago, before the previous barrier.
    float* pt = part + p.half(s) * (V * kMaxWaves);
    if (butterfly_writer<V>(lane)) pt[wave * V + butterfly_index<V>(lane)] = acc[0];
    __syncthreads();
    for (int t = threadIdx.x; t < R * M; t += block_threads()) {
      const int r = t / M, m = t % M;
      const int j = j0 + r;
      if (j < I) {
        float gs = 0.f, us = 0.f;
        for (int i = 0; i < nw; ++i) {
          gs += pt[i * V + t];
          us += pt[i * V + R * M + t];
        }
        float gsc = sg[0], usc = su[0];
#pragma unroll
        for (int q = 1; q < R; ++q)
          if (r == q) gsc = sg[q], usc = su[q];
        mid[m * (int64_t)I + j] = swiglu_out<T>(gs * gsc, us * usc);
      }
    }
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
  };
  stream_steps(p.total, a, b, issue, consume);
}

// Relayout form of the MFMA gate/up for M >= kFp8MfmaMinM (M padded to 16). A
// lane loads 16 codes (one 16-byte load) of row lane/8 (+8 for the second load)
// at K chunk lane%8 of a 128-wide unit, decodes them to two 8-element chunks of
// the activation type (exact values) and stores those to the wave's
// XOR-swizzled LDS tile exactly where the fp16 relayout kernel (gemv.hip) stores
// a loaded chunk; the A reads, B (x) loads and MFMAs are that kernel's, and the
// channel scale is applied to the sums.
template <typename T>
__device__ __forceinline__ void fp8x16_to_tile(const u32x4& w, u32x4& c0, u32x4& c1) {
  uint32_t h[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) fp8x4_to_pairs<T>(w[i], h[2 * i], h[2 * i + 1]);
  c0 = u32x4{h[0], h[1], h[2], h[3]};
  c1 = u32x4{h[4], h[5], h[6], h[7]};
}

// Registers of one 16x128 unit of the MFMA forms: S weight sets (gate/up: 2) of
// two 16-byte code loads each, and the four B (x) fragments.
template <typename T, int S>
struct UnitRegs8 {
  u32x4 v[S][2];
  typename Vec8<T>::type b[4];
};

// Loads of unit u, all unconditional: a lane whose K chunk is past K reads its
// row's first 16 codes instead (masked when staged), a B fragment past K its x
// row's first fragment (masked in unit_b). `wl` are code row bases (rows past N
// clamped by the caller to row 0), `xr` the lane's x row.
template <typename T, int S, bool LOADB = true>
__device__ __forceinline__ void load_unit8(UnitRegs8<T, S>& q, const uint8_t* const (&wl)[S][2],
                                           const T* xr, int u, int lchunk, int g, int K) {
  const int k = u * kUnit + lchunk * 16;
  const int kc = k < K ? k : 0;
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int j = 0; j < 2; ++j) q.v[s][j] = load16_nt(wl[s][j] + kc);
  if constexpr (LOADB) {
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      const int kb = u * kUnit + (s2 * 4 + g) * 8;
      q.b[s2] = load8<T>(xr + (kb < K ? kb : 0));
    }
  }
}

// Decode a unit's codes (zeros past K) into the wave's LDS tile and read back
// the MFMA A fragments.
template <typename T>
__device__ __forceinline__ void stage_unit8(const u32x4 (&v)[2], u32x4* tile, int lrow, int lchunk,
                                            int u, int K, int r, int g,
                                            typename Vec8<T>::type (&a)[4]) {
  const bool in = u * kUnit + lchunk * 16 < K;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    u32x4 c0, c1;
    fp8x16_to_tile<T>(in ? v[i] : u32x4{0, 0, 0, 0}, c0, c1);
    const int row = 8 * i + lrow;
    tile[row * 16 + ((2 * lchunk) ^ row)] = c0;
    tile[row * 16 + ((2 * lchunk + 1) ^ row)] = c1;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) a[s2] = __builtin_bit_cast(typename Vec8<T>::type, tile[r * 16 + ((s2 * 4 + g) ^ r)]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Pre-attention QKV with fp8 weights for M < 5: the fp16 fused QKV kernel's
// structure (RMSNorm prologue staged in LDS, 4 weight rows per tile placed by
// TileRows<4>, the step pipeline of stream_steps, RoPE of the
// rotated tiles in the epilogue) with the fp8 GEMV's 16 codes per lane and step.
template <int R>
struct Rows8Regs {
  u32x4 v[R];
};

template <int R>
__device__ __forceinline__ void load_tile_rows8(Rows8Regs<R>& b, const uint8_t* w, const Rope& rp,
                                                const StepPlan& p, int s, int H, int N) {
  const TileRows<R> tr(rp, p.tile(s));
  const int k = p.k(s);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = tr.row(r);
    const bool ok = n < N && k < H;
    b.v[r] = load16_nt(ok ? w + n * H + k : w);
  }
}

template <typename T, int M, int R, bool REGS>
__global__ __launch_bounds__(kMaxWaves * kWave) void qkv_fp8_kernel(
    T* y, const T* hidden, const void* nwp, int nw_dtype, const uint8_t* w, const float* wscale,
    int H, int N, float eps, int tiles, Epi e, Rope rp) {
  typedef typename Vec8<T>::type V8;
  constexpr int V = pow2_ceil(R * M);
  extern __shared__ __align__(16) unsigned char smem[];
  const int XS = xs_stride(H);
  T* xs = reinterpret_cast<T*>(smem);
  float* part = reinterpret_cast<float*>(smem + (size_t)M * XS * sizeof(T));
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = block_threads() / kWave;
  const StepPlan p(tiles, H, nw * kChunk8, (wave * kWave + lane) * 16);

  NormRegs<T, M, kNormRegRows(M)> nr;
  if constexpr (REGS) norm_load(nr, hidden, nwp, nw_dtype, M, H);
  Rows8Regs<R> a, b;
  load_tile_rows8<R>(a, w, rp, p, 0, H, N);
  if constexpr (REGS)
    norm_store(nr, xs, part, nw_dtype, M, H, eps);
  else
    stage_normed<T, M>(xs, part, hidden, nwp, nw_dtype, M, H, eps);

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  auto issue = [&](Rows8Regs<R>& buf, int s) { load_tile_rows8<R>(buf, w, rp, p, s, H, N); };
  auto consume = [&](const Rows8Regs<R>& buf, int s) {
    const int k = p.k(s);
    if (k < H) {
      V8 xa[M], xb[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        xa[m] = load8<T>(xs + m * XS + k);
        xb[m] = load8<T>(xs + m * XS + k + 8);
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r * M + m] = dot_fp8x16<T>(buf.v[r], xa[m], xb[m], acc[r * M + m]);
    }
    if (!p.last(s)) return;
    butterfly_sum<V>(acc, lane);
    // Consecutive tiles alternate halves of `part`, so one barrier suffices: the
    // half written here was last read two tiles ago, before the previous barrier.
    float* pt = part + p.half(s) * (V * kMaxWaves);
    if (butterfly_writer<V>(lane)) pt[wave * V + butterfly_index<V>(lane)] = acc[0];
    __syncthreads();
    qkv_tile_out<T, M, R>(y, pt, V, nw, TileRows<R>(rp, p.tile(s)), e, rp, RowScale{wscale}, N);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
  };
  stream_steps(p.total, a, b, issue, consume);
}

// Gate/up + SwiGLU in the same form (M >= 5): 16 gate and the matching 16 up
// rows per workgroup, x the raw hidden state, normalised inside the kernel as
// in mlp_gate_up_relayout_kernel's SS form (gemv.hip): the norm weight staged
// in LDS, inv[m] from the producer's row sums of squares (RowSq) or, with FX,
// from a pass over x in the prologue, each B fragment round(x * inv * w).
// Held to the VGPRs of three waves per SIMD. Two waves per workgroup (six per
// CU: all 896 of Llama-3-8B's resident at once); four for the form the decode
// step runs (HALF with the producer's sums), whose 126 VGPRs leave four waves
// per SIMD, so its 896 four-wave workgroups are all resident too and each CU
// keeps twice the units in flight (M=8 step: 26.7 -> 26.2 us).
// HALF (M <= 8): the activation fragments in the half-B form (load_b_half).
// SPLIT: 8 gate rows and their 8 up rows in one 16-row set, paired in the
// epilogue as in gemv.hip's gate_up_relayout_tile; these take the rows past the
// last whole round of 16 + 16 tiles over the CUs (relayout_grid).
template <bool HALF, bool FX>
constexpr int fp8_ss_waves() { return HALF && !FX ? 4 : 2; }
template <typename T, bool HALF, bool FX, bool SPLIT>
__device__ __forceinline__ void gate_up_fp8_relayout_tile(f32x4* part, u32x4 (*tiles)[256], int64_t j0, T* mid,
                                                          const T* x, const uint8_t* wgu, const float* gu_scale,
                                                          int M, int H, int I, const void* nwp, int nw_dtype,
                                                          float eps, const RowSq& rq) {
  typedef typename Vec8<T>::type V8;
  constexpr int LW = fp8_ss_waves<HALF, FX>();
  constexpr int S = SPLIT ? 1 : 2;  // weight sets per unit
  extern __shared__ float norm_lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = block_threads() / kWave;
  const int r = lane & 15, g = lane >> 4;
  const int hi = r >= 8, xrow = HALF ? half_b_row(r) : r;
  const T* xr = x + (xrow < M ? xrow : 0) * (int64_t)H;  // rows past M: columns never stored
  const int lrow = lane >> 3, lchunk = lane & 7;
  const uint8_t* wl[S][2];  // [gate, up][row lrow, lrow + 8] bases; SPLIT: gate row lrow, its up row
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if constexpr (SPLIT) {
      const int64_t j = j0 + lrow;
      const int64_t jc = j < I ? j : 0;
      wl[0][i] = wgu + (i == 0 ? jc : I + jc) * H;
    } else {
      const int64_t j = j0 + 8 * i + lrow;
      const int64_t jc = j < I ? j : 0;
      wl[0][i] = wgu + jc * H;
      wl[S - 1][i] = wgu + (I + jc) * H;
    }
  }
  u32x4* tile = tiles[wave];
  f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
  const int units = (H + kUnit - 1) / kUnit;
  const int mine = wave < units ? (units - wave + nw - 1) / nw : 0;
  const int off = sweep_offset(units);
  auto issue = [&](UnitRegs8<T, S>& q, int i) {
    const int u = sweep_unit(wave, i, nw, off, units);
    load_unit8<T, S, !HALF>(q, wl, xr, u, lchunk, g, H);
    if constexpr (HALF) load_b_half<T>(q.b, xr, u, g, hi, H);
  };
  float rinv = 0.f;
  // fragment s2's B: the normalised activations, zero past K
  auto frag = [&](const V8& raw, int u, int s2) {
    const f32x4* wk = reinterpret_cast<const f32x4*>(norm_lds + u * kUnit + (s2 * 4 + g) * 8);
    const V8 xb = __builtin_bit_cast(V8, norm_frag<T>(__builtin_bit_cast(u32x4, raw), rinv,
                                                      __builtin_bit_cast(u32x4, wk[0]),
                                                      __builtin_bit_cast(u32x4, wk[1])));
    return unit_b(xb, u, s2, g, H);
  };
  auto consume = [&](const UnitRegs8<T, S>& q, int i) {
    const int u = sweep_unit(wave, i, nw, off, units);
    V8 a[4], c[4];
    stage_unit8<T>(q.v[0], tile, lrow, lchunk, u, H, r, g, a);
    if constexpr (!SPLIT) stage_unit8<T>(q.v[S - 1], tile, lrow, lchunk, u, H, r, g, c);
    if constexpr (HALF) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const V8 own = frag(q.b[p], u, 2 * p + hi);
        const V8 oth = __builtin_bit_cast(V8, mirror16(__builtin_bit_cast(u32x4, own)));
        ag = mfma16(a[2 * p], own, ag);
        if constexpr (!SPLIT) au = mfma16(c[2 * p], own, au);
        ag = mfma16(a[2 * p + 1], oth, ag);
        if constexpr (!SPLIT) au = mfma16(c[2 * p + 1], oth, au);
      }
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        const V8 b = frag(q.b[s2], u, s2);
        ag = mfma16(a[s2], b, ag);
        if constexpr (!SPLIT) au = mfma16(c[s2], b, au);
      }
    }
  };
  UnitRegs8<T, S> qa, qb;
  {  // the first two units' loads fly while the prologue runs
    float* inv = norm_lds + units * kUnit;
    norm_prologue<T, HALF ? 8 : 16, FX, LW * kWave>(norm_lds, inv, inv + 16, nwp, nw_dtype, x, H, M, H,
                                                             units * kUnit, eps, rq, [&] {
                                                               if (mine > 0) issue(qa, 0);
                                                               if (mine > 1) issue(qb, 1);
                                                             });
    rinv = inv[xrow];
  }
  stream_steps_issued2(mine, qa, qb, issue, consume);
  if constexpr (SPLIT) {  // one reduction: lane t < 32 adds the gate sums of t, the up sums of t + 32
    part[wave * kWave + lane] = ag;
    __syncthreads();
    if (threadIdx.x < 32) {
      f32x4 sg = part[threadIdx.x], su = part[threadIdx.x + 32];
      for (int i = 1; i < nw; ++i) {
        sg += part[i * kWave + threadIdx.x];
        su += part[i * kWave + threadIdx.x + 32];
      }
      const int m = threadIdx.x & 15;
      const int nb = (threadIdx.x >> 4) * 4;
      if (m < M) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t jj = j0 + nb + i;
          if (jj < I)
            mid[m * (int64_t)I + jj] = swiglu_out<T>(sg[i] * gu_scale[jj], su[i] * gu_scale[I + jj]);
        }
      }
    }
    return;
  }
  part[wave * kWave + lane] = ag;
  __syncthreads();
  f32x4 sg = {0.f, 0.f, 0.f, 0.f};
  if (threadIdx.x < kWave)
    for (int i = 0; i < nw; ++i) sg += part[i * kWave + threadIdx.x];
  __syncthreads();
  part[wave * kWave + lane] = au;
  __syncthreads();
  if (threadIdx.x < kWave) {
    f32x4 su = part[threadIdx.x];
    for (int i = 1; i < nw; ++i) su += part[i * kWave + threadIdx.x];
    const int m = threadIdx.x & 15;
    const int nb = (threadIdx.x >> 4) * 4;
    if (m < M) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t jj = j0 + nb + i;
        if (jj < I)
          mid[m * (int64_t)I + jj] =
              swiglu_out<T>(sg[i] * gu_scale[jj], su[i] * gu_scale[I + jj]);
      }
    }
  }
}

// The gate/up launch: workgroup b < big takes 16 gate + 16 up rows from 16 b;
// with MIX the rest take 8 + 8 rows each after those (relayout_grid).
template <typename T, bool HALF, bool FX, bool MIX = false>
__global__ __launch_bounds__((fp8_ss_waves<HALF, FX>() * kWave), 3) void mlp_gate_up_fp8_relayout_kernel(
    T* mid, const T* x, const uint8_t* wgu, const float* gu_scale, int M, int H, int I, const void* nwp,
    int nw_dtype, float eps, RowSq rq, int big) {
  constexpr int LW = fp8_ss_waves<HALF, FX>();
  __shared__ f32x4 part[LW * kWave];
  __shared__ u32x4 tiles[LW][256];
  const int b = (int)blockIdx.x;
  if constexpr (MIX) {
    if (b >= big) {
      gate_up_fp8_relayout_tile<T, HALF, FX, true>(part, tiles, (int64_t)big * 16 + (int64_t)(b - big) * 8, mid, x,
                                                   wgu, gu_scale, M, H, I, nwp, nw_dtype, eps, rq);
      return;
    }
  }
  gate_up_fp8_relayout_tile<T, HALF, FX, false>(part, tiles, (int64_t)b * 16, mid, x, wgu, gu_scale, M, H, I, nwp,
                                                nw_dtype, eps, rq);
}

namespace {

template <int M> struct Fp8Rows { static constexpr int R = M <= 8 ? 4 : 2; };
// Four gate + four up rows per tile with two workgroups per CU up to 4 rows
// (Llama-3-8B widths: M=1 20.2 us against 20.8 for two rows at four per CU,
// M=2 20.9 against 22.0); above, two rows, which keeps 2*R*M sums per lane
// within the butterfly's 64.
template <int M> struct Fp8MlpRows { static constexpr int R = M <= 4 ? 4 : 2; };
template <int M> struct Fp8MlpPerCu { static constexpr int P = 2; };

// Fused QKV: R rows per tile (R/2 rotate-half pairs in a rotated tile); eight
// up to 2 rows (Llama-3-8B widths, M=1: 9.1 against 9.7 us for four).
template <int M> struct Fp8QkvRows { static constexpr int R = M <= 2 ? 8 : 4; };

// From this many rows the fp8 GEMV and MLP take the MFMA (relayout) forms.
constexpr int kFp8MfmaMinM = 5;


// The persistent fp8 SIMT kernel (fp8_px_kernel): the fewest 1024-element
// chunks per lane (1, 2 or 4) that keep K within eight waves, four rows per
// tile where the registers hold them, else two; one workgroup per CU unless
// N >= 8*M*CUs (each workgroup first reads M*K activations, as many bytes as
// 2*M rows of codes). Used for M in [kFp8PxMinM, kFp8PxMaxM], where it beats
// the per-tile SIMT kernels (Llama-3-8B shapes, M = 2 / 4: N = K = 4096 5.44 /
// 5.86 us against 5.56 / 6.51; N = 6144 6.56 / 7.19 against 7.11 / 8.36;
// K = 14336 12.8 / 12.9 against 13.4 / 16.1; N = 28672 20.6 / 22.2 against
// 21.7 / 28.2; the fused QKV at M = 4 10.7 against 12.3). From 5 rows its
// decode and v_dot2 work make it slower than the MFMA kernel (M = 8, N = 6144:
// 9.1 against 8.6 us); at one row the two SIMT forms tie.
constexpr int kFp8PxMinM = 2;
constexpr int kFp8PxMaxM = 4;
__host__ __device__ constexpr bool fp8_px_regs_ok(int M, int R, int cpl) {
  return cpl * M * 8 + 8 * R * cpl + pow2_ceil(R * M) <= 224;
}
inline int fp8_px_waves(int K, int cpl) {
  const int chunks = (K + kChunk8 - 1) / kChunk8;
  return (chunks + cpl - 1) / cpl;
}
inline int fp8_px_grid(int N, int M, int tiles) {
  const int cus = device_cus();
  const int grid = (N < 8 * M * cus ? 1 : 2) * cus;
  return grid < tiles ? grid : tiles;
}
template <int M>
bool fp8_px_shape(int N, int K, int& rows, int& cpl) {
  if (K <= 0) return false;
  const int chunks = (K + kChunk8 - 1) / kChunk8;
  cpl = chunks <= kMaxWaves ? 1 : chunks <= 2 * kMaxWaves ? 2 : 4;
  if (fp8_px_waves(K, cpl) > kMaxWaves) return false;
  rows = fp8_px_regs_ok(M, 4, cpl) ? 4 : 2;
  if (!fp8_px_regs_ok(M, rows, cpl)) return false;
  const int tiles = (N + rows - 1) / rows + 1;  // a QKV may split its rows into one more tile
  const int grid = fp8_px_grid(N, M, tiles);
  const int per = (tiles + grid - 1) / grid;
  const size_t lds = sizeof(float) * ((size_t)per * fp8_px_waves(K, cpl) * pow2_ceil(rows * M) +
                                      kMaxWaves * pow2_ceil(M) + pow2_ceil(M));
  return lds <= kMaxLds / 2;
}

template <typename T, int M, int R, int CPL, int MODE>
int launch_fp8_px_r(void* y, const void* x, const uint8_t* w, const float* s, int N, int K, int64_t sxm,
                    int64_t swn, int64_t sym, int64_t syn, const Epi& e, const void* nwp, int nw_dtype,
                    float eps, Rope rp, hipStream_t st) {
  constexpr int V = pow2_ceil(R * M), MP = pow2_ceil(M);
  const int nwv = fp8_px_waves(K, CPL);
  int tiles = (N + R - 1) / R;
  if constexpr (MODE == kPxQkv) {
    rp.tiles = rp.cols / R;
    tiles = rp.tiles + (N - rp.cols + R - 1) / R;
  } else if constexpr (MODE == kPxGateUp) {
    tiles = (N / 2 + R / 2 - 1) / (R / 2);
  }
  const int grid = fp8_px_grid(N, M, tiles);
  const int per = (tiles + grid - 1) / grid;
  const size_t lds = sizeof(float) * ((size_t)per * nwv * V + kMaxWaves * MP + MP);
  auto kernel = fp8_px_kernel<T, M, R, CPL, MODE>;
  if (!allow_lds(kernel, lds)) return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", lds);
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(nwv * kWave), lds, st, static_cast<T*>(y), static_cast<const T*>(x),
                     w, s, N, K, sxm, swn, sym, syn, e, tiles, nwp, nw_dtype, eps, rp);
  return FD_OK;
}

template <typename T, int M, int MODE>
int launch_fp8_px(void* y, const void* x, const uint8_t* w, const float* s, int N, int K, int64_t sxm,
                  int64_t swn, int64_t sym, int64_t syn, const Epi& e, const void* nwp, int nw_dtype, float eps,
                  const Rope& rp, hipStream_t st) {
  int rows = 0, cpl = 0;
  if (!fp8_px_shape<M>(N, K, rows, cpl))
    return set_error(FD_EUNSUPPORTED, "the persistent fp8 SIMT kernel does not take K = %d", K);
  auto go = [&](auto rtag, auto ctag) -> int {
    constexpr int RR = decltype(rtag)::value, CC = decltype(ctag)::value;
    if constexpr (fp8_px_regs_ok(M, RR, CC))
      return launch_fp8_px_r<T, M, RR, CC, MODE>(y, x, w, s, N, K, sxm, swn, sym, syn, e, nwp, nw_dtype, eps, rp,
                                                st);
    return set_error(FD_EUNSUPPORTED, "the persistent fp8 SIMT kernel's registers do not hold M = %d", M);
  };
  using R2 = std::integral_constant<int, 2>;
  using R4 = std::integral_constant<int, 4>;
  using C1 = std::integral_constant<int, 1>;
  using C2 = std::integral_constant<int, 2>;
  using C4 = std::integral_constant<int, 4>;
  if (rows == 4) return cpl == 1 ? go(R4{}, C1{}) : cpl == 2 ? go(R4{}, C2{}) : go(R4{}, C4{});
  return cpl == 1 ? go(R2{}, C1{}) : cpl == 2 ? go(R2{}, C2{}) : go(R2{}, C4{});
}

inline bool fp8_px_takes(int M, int N, int K) {
  if (M < kFp8PxMinM || M > kFp8PxMaxM) return false;
  int rows = 0, cpl = 0;
  switch (M) {
#define FD_CASE(MM) \
  case MM: return fp8_px_shape<MM>(N, K, rows, cpl);
    FD_CASE(2) FD_CASE(3) FD_CASE(4)
#undef FD_CASE
    default: return false;
  }
}

template <typename T, int MODE>
int launch_fp8_px_m(int M, void* y, const void* x, const uint8_t* w, const float* s, int N, int K, int64_t sxm,
                    int64_t swn, int64_t sym, int64_t syn, const Epi& e, const void* nwp, int nw_dtype, float eps,
                    const Rope& rp, hipStream_t st) {
  switch (M) {
#define FD_CASE(MM) \
  case MM:                                                                                                     \
    return launch_fp8_px<T, MM, MODE>(y, x, w, s, N, K, sxm, swn, sym, syn, e, nwp, nw_dtype, eps, rp, st);
    FD_CASE(2) FD_CASE(3) FD_CASE(4)
#undef FD_CASE
    default: return set_error(FD_EINVAL, "the persistent fp8 SIMT kernel takes M in [%d, %d]", kFp8PxMinM,
                              kFp8PxMaxM);
  }
}

// The MFMA form (kFp8MfmaMinM rows and up): the DMA GEMV of fd_dma.h. `rp`
// (fused QKV): tiles placed by TileRows<16> with RoPE in the epilogue; `fold`:
// the RMSNorm of x folded in (x = raw activations).
template <typename T>
int launch_gemv_fp8_mfma(int M, void* y, const void* x, const uint8_t* w, const float* s, int N,
                         int K, int64_t sxm, int64_t swn, int64_t sym, int64_t syn, const Epi& e,
                         hipStream_t st, const Rope* rp = nullptr, const FoldNorm* fold = nullptr) {
  const FoldNorm nofold{nullptr, FD_F32, 0.f};
  const Rope none{};
  const unsigned blocks =
      rp ? (unsigned)(rp->tiles + (N - rp->cols + 15) / 16) : (unsigned)((N + 15) / 16);
  // The fused QKV at 5-8 rows with the producer's row sums: eight waves, two
  // units in flight each, where K gives every wave a unit (Llama-3-8B widths,
  // M = 5 / 8: 10.3 / 10.9 -> 10.1 / 10.6 us; in the decode step 11.6 -> 11.2).
  // Not with 16 rows, whose larger B tiles would leave one such workgroup per
  // CU (13.2 -> 16.9), nor where the prologue sums x itself (M = 8: 11.9 -> 13.0)
  if (rp && fold && fold->sq.p && dma_rows(M) <= 8 && (K + kUnit - 1) / kUnit >= 8)
    return launch_dma_rows<T, uint8_t, 8, 2, EPI_ROPE, true>(blocks, y, x, w, s, M, N, K, sxm, swn, sym, syn, e,
                                                             *rp, *fold, st);
  if (rp && fold)
    return launch_dma_default<T, uint8_t, EPI_ROPE, true>(blocks, y, x, w, s, M, N, K, sxm, swn, sym, syn, e,
                                                          *rp, *fold, st);
  if (rp)
    return launch_dma_default<T, uint8_t, EPI_ROPE, false>(blocks, y, x, w, s, M, N, K, sxm, swn, sym, syn, e,
                                                           *rp, nofold, st);
  if ((K + kUnit - 1) / kUnit < 4)
    return launch_dma_rows<T, uint8_t, 2, 2, EPI_PLAIN, false>(blocks, y, x, w, s, M, N, K, sxm, swn, sym, syn,
                                                               e, none, nofold, st);
  // One tile per CU or fewer (N = 4096): eight waves, two units in flight each,
  // so every SIMD has two waves; up to two rounds: four waves, three units in
  // flight; wider layers: four waves, two units (Llama-3-8B widths, M=8:
  // N=4096 K=14336 14.4 us against 14.9 for 4 x 3 and 17.0 for 4 x 2; N=6144
  // 9.5 with 4 x 3; N=28672 K=4096 26.6 against 27.6 for 4 x 3; the relayout
  // kernel this replaced: 15.6, 11.0 and 29.8). A launch that also writes the
  // row sums for the next norm (the decode step's O and down projections, with
  // the residual as row_add) runs four waves with four units in flight there
  // (M=8: N = K = 4096 7.0 -> 6.6 us, K = 14336 14.3 -> 13.8; without the sums
  // the two shapes tie).
  if (blocks <= (unsigned)device_cus() && e.ss && (K + kUnit - 1) / kUnit >= 16)
    return launch_dma_rows<T, uint8_t, 4, 4, EPI_PLAIN, false>(blocks, y, x, w, s, M, N, K, sxm, swn, sym, syn,
                                                               e, none, nofold, st);
  if (blocks <= (unsigned)device_cus())
    return launch_dma_rows<T, uint8_t, 8, 2, EPI_PLAIN, false>(blocks, y, x, w, s, M, N, K, sxm, swn, sym, syn,
                                                               e, none, nofold, st);
  if (blocks <= 2u * (unsigned)device_cus())
    return launch_dma_rows<T, uint8_t, 4, 3, EPI_PLAIN, false>(blocks, y, x, w, s, M, N, K, sxm, swn, sym, syn,
                                                               e, none, nofold, st);
  return launch_dma_rows<T, uint8_t, 4, 2, EPI_PLAIN, false>(blocks, y, x, w, s, M, N, K, sxm, swn, sym, syn, e,
                                                             none, nofold, st);
}

template <typename T, int M>
void launch_gemv_fp8(void* y, const void* x, const uint8_t* w, const float* s, int N, int K,
                     int64_t sxm, int64_t swn, int64_t sym, int64_t syn, const Epi& e,
                     hipStream_t st) {
  constexpr int R = Fp8Rows<M>::R;
  const int nw = pick_waves((K + kChunk8 - 1) / kChunk8);
  hipLaunchKernelGGL((gemv_fp8_kernel<T, M, R>), dim3((unsigned)((N + R - 1) / R)),
                     dim3(nw * kWave), 0, st, static_cast<T*>(y), static_cast<const T*>(x), w, s,
                     N, K, sxm, swn, sym, syn, e);
}

template <typename T>
int launch_gemv_fp8_m(int M, void* y, const void* x, const uint8_t* w, const float* s, int N,
                      int K, int64_t sxm, int64_t swn, int64_t sym, int64_t syn, const Epi& e,
                      hipStream_t st) {
  if (M >= kFp8MfmaMinM) return launch_gemv_fp8_mfma<T>(M, y, x, w, s, N, K, sxm, swn, sym, syn, e, st);
  switch (M) {
#define FD_CASE(MM) \
  case MM: launch_gemv_fp8<T, MM>(y, x, w, s, N, K, sxm, swn, sym, syn, e, st); break;
    FD_CASE(1) FD_CASE(2) FD_CASE(3) FD_CASE(4) FD_CASE(5) FD_CASE(6) FD_CASE(7) FD_CASE(8)
    FD_CASE(9) FD_CASE(10) FD_CASE(11) FD_CASE(12) FD_CASE(13) FD_CASE(14) FD_CASE(15)
    FD_CASE(16)
#undef FD_CASE
    default: break;
  }
  return FD_OK;
}

template <typename T, int M>
int launch_mlp_fp8(void* mid, const void* hidden, const void* nw, int nw_dtype,
                   const uint8_t* wgu, const float* s, int H, int I, float eps, hipStream_t st) {
  constexpr int R = Fp8MlpRows<M>::R;
  constexpr int V = pow2_ceil(2 * R * M);
  const int nwv0 = pick_waves((H + kChunk8 - 1) / kChunk8);
  const int nwv = M > kNormRegMaxM && nwv0 > 4 ? 4 : nwv0;
  const size_t lds = fused_lds(M, H, sizeof(T), V);
  if (lds > kMaxLds) return set_error(FD_EUNSUPPORTED, "M*H too large for the LDS stage");
  const int tiles = (I + R - 1) / R;
  const int grid = fused_grid(tiles, lds, Fp8MlpPerCu<M>::P);
  auto launch = [&](auto kernel) {
    if (!allow_lds(kernel, lds))
      return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", lds);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(nwv * kWave), lds, st, static_cast<T*>(mid),
                       static_cast<const T*>(hidden), nw, nw_dtype, wgu, s, H, I, eps, tiles);
    return (int)FD_OK;
  };
  if constexpr (M <= kNormRegMaxM) {
    if (norm_in_regs(M, H, nwv * kWave)) return launch(mlp_gate_up_fp8_kernel<T, M, R, true>);
  }
  return launch(mlp_gate_up_fp8_kernel<T, M, R, false>);
}

template <typename T>
int launch_mlp_fp8_m(int M, void* mid, const void* hidden, const void* nw, int nw_dtype,
                     const uint8_t* wgu, const float* s, int H, int I, float eps, hipStream_t st) {
  switch (M) {
#define FD_CASE(MM) \
  case MM: return launch_mlp_fp8<T, MM>(mid, hidden, nw, nw_dtype, wgu, s, H, I, eps, st);
    FD_CASE(1) FD_CASE(2) FD_CASE(3) FD_CASE(4) FD_CASE(5) FD_CASE(6) FD_CASE(7) FD_CASE(8)
    FD_CASE(9) FD_CASE(10) FD_CASE(11) FD_CASE(12) FD_CASE(13) FD_CASE(14) FD_CASE(15)
    FD_CASE(16)
#undef FD_CASE
    default: return set_error(FD_EINVAL, "M must be in [1, 16]");
  }
}

// Fused QKV, M < kFp8MfmaMinM: up to four waves and every tile resident at once
// (the fp16 QKV launch shape).
template <typename T, int M>
int launch_qkv_fp8(void* y, const void* hidden, const void* nw, int nw_dtype, const uint8_t* w,
                   const float* s, int H, int N, float eps, const Epi& e, const Rope& rp_in,
                   hipStream_t st) {
  constexpr int R = Fp8QkvRows<M>::R;
  constexpr int V = pow2_ceil(R * M);
  const int nwv0 = pick_waves((H + kChunk8 - 1) / kChunk8);
  const int nwv = nwv0 > 4 ? 4 : nwv0;
  const size_t lds = fused_lds(M, H, sizeof(T), V);
  if (lds > kMaxLds) return set_error(FD_EUNSUPPORTED, "M*H too large for the LDS stage");
  Rope rp = rp_in;
  rp.tiles = rp.cols / R;
  const int tiles = rp.tiles + (N - rp.cols + R - 1) / R;
  const int grid = fused_grid(tiles, lds, 8);
  auto launch = [&](auto kernel) {
    if (!allow_lds(kernel, lds))
      return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", lds);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(nwv * kWave), lds, st, static_cast<T*>(y),
                       static_cast<const T*>(hidden), nw, nw_dtype, w, s, H, N, eps, tiles, e, rp);
    return (int)FD_OK;
  };
  if constexpr (M <= kNormRegMaxM) {
    if (norm_in_regs(M, H, nwv * kWave)) return launch(qkv_fp8_kernel<T, M, R, true>);
  }
  return launch(qkv_fp8_kernel<T, M, R, false>);
}

template <typename T>
int launch_qkv_fp8_m(int M, void* y, const void* hidden, const void* nw, int nw_dtype,
                     const uint8_t* w, const float* s, int H, int N, float eps, const Epi& e,
                     const Rope& rp, hipStream_t st) {
  switch (M) {
#define FD_CASE(MM) \
  case MM: return launch_qkv_fp8<T, MM>(y, hidden, nw, nw_dtype, w, s, H, N, eps, e, rp, st);
    FD_CASE(1) FD_CASE(2) FD_CASE(3) FD_CASE(4)
#undef FD_CASE
    default: return set_error(FD_EINVAL, "the SIMT fp8 QKV covers M < %d", kFp8MfmaMinM);
  }
}

}  // namespace
}  // namespace fd

namespace fd {
namespace {

int linear_fp8_entry(void* y, const void* x, const void* w8, const float* w_scale, const void* bias,
                     int bias_dtype, const void* row_add, int row_dtype, int64_t M, int64_t N, int64_t K,
                     int64_t sxm, int64_t swn, int64_t sb, int64_t srm, int64_t srn, int64_t sym, int64_t syn,
                     int act_dtype, float* ss_out, void* stream) {
  if (!check_act_dtype(act_dtype)) return FD_EINVAL;
  if (M < 0 || N < 0 || K < 0) return set_error(FD_EINVAL, "negative size");
  if (M > 16) return set_error(FD_EINVAL, "the fp8 GEMV covers M <= 16");
  if (sxm < 0 || swn < 0 || sb < 0 || srm < 0 || srn < 0 || sym < 0 || syn < 0)
    return set_error(FD_EINVAL, "negative stride");
  if (bias && bias_dtype != act_dtype && bias_dtype != FD_F32)
    return set_error(FD_EINVAL, "bias must match x or be float32");
  if (row_add && !check_any_dtype(row_dtype, "row_dtype")) return FD_EINVAL;
  if (M == 0 || N == 0) return FD_OK;
  // K = 0 reads neither operand (an empty torch tensor's pointer is null)
  if (!y || !w_scale || ((!x || !w8) && K > 0)) return set_error(FD_EINVAL, "null pointer argument");
  if (K % 16 != 0 || (N > 1 && swn % 16 != 0) || (M > 1 && sxm % 8 != 0))
    return set_error(FD_EUNSUPPORTED, "the fp8 GEMV needs K %% 16 == 0 and 16-byte aligned rows");
  if (!aligned16(x) || !aligned16(w8)) return set_error(FD_EUNSUPPORTED, "operands must be 16-byte aligned");
  if (N > 0x7fffffffLL || K > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "too large");
  Epi e;
  e.bias = bias;
  e.bias_dtype = bias_dtype;
  e.sb = sb;
  e.row = row_add;
  e.row_dtype = row_dtype;
  e.srm = srm;
  e.srn = srn;
  e.ss = ss_out;  // the MFMA form writes it (the caller checked M)
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint8_t* w = static_cast<const uint8_t*>(w8);
  int rc;
  if (!ss_out && fp8_px_takes((int)M, (int)N, (int)K)) {
    const Rope none{};
    rc = act_dtype == FD_F16
             ? launch_fp8_px_m<f16, kPxGemv>((int)M, y, x, w, w_scale, (int)N, (int)K, sxm, swn, sym, syn, e, nullptr,
                                          FD_F32, 0.f, none, st)
             : launch_fp8_px_m<bf16, kPxGemv>((int)M, y, x, w, w_scale, (int)N, (int)K, sxm, swn, sym, syn, e,
                                           nullptr, FD_F32, 0.f, none, st);
  } else {
    rc = act_dtype == FD_F16
             ? launch_gemv_fp8_m<f16>((int)M, y, x, w, w_scale, (int)N, (int)K, sxm, swn, sym, syn, e, st)
             : launch_gemv_fp8_m<bf16>((int)M, y, x, w, w_scale, (int)N, (int)K, sxm, swn, sym, syn, e, st);
  }
  if (rc != FD_OK) return rc;
  return check_launch();
}

}  // namespace
}  // namespace fd

extern "C" int fd_linear_fp8(void* y, const void* x, const void* w8, const float* w_scale,
                             const void* bias, int bias_dtype, const void* row_add, int row_dtype,
                             int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t swn,
                             int64_t sb, int64_t srm, int64_t srn, int64_t sym, int64_t syn,
                             int act_dtype, void* stream) {
  return fd::linear_fp8_entry(y, x, w8, w_scale, bias, bias_dtype, row_add, row_dtype, M, N, K, sxm, swn, sb,
                              srm, srn, sym, syn, act_dtype, nullptr, stream);
}

extern "C" int fd_linear_fp8_sumsq(void* y, const void* x, const void* w8, const float* w_scale,
                                   const void* bias, int bias_dtype, const void* row_add, int row_dtype,
                                   int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t swn, int64_t sb,
                                   int64_t srm, int64_t srn, int64_t sym, int64_t syn, int act_dtype,
                                   float* ss_out, void* stream) {
  using namespace fd;
  if (!ss_out) return set_error(FD_EINVAL, "null pointer argument");
  const int rc = check_sumsq(M >= kFp8MfmaMinM && M <= 16, nullptr, 0, 0, ss_out);
  if (rc != FD_OK) return rc;
  return linear_fp8_entry(y, x, w8, w_scale, bias, bias_dtype, row_add, row_dtype, M, N, K, sxm, swn, sb, srm,
                          srn, sym, syn, act_dtype, ss_out, stream);
}

namespace fd {
namespace {

int post_attn_mlp_fp8_entry(void* y, void* mid, const void* hidden, const void* norm_w, int norm_w_dtype,
                            const void* w_gate_up8, const float* gate_up_scale, const void* w_down8,
                            const float* down_scale, int64_t M, int64_t H, int64_t I, float eps, int act_dtype,
                            const RowSq* rq, float* ss_out, void* stream) {
  if (!check_act_dtype(act_dtype) || !check_any_dtype(norm_w_dtype, "norm_w_dtype"))
    return FD_EINVAL;
  if (M < 0 || M > 16) return set_error(FD_EINVAL, "M must be in [0, 16]");
  if (H <= 0 || I <= 0) return set_error(FD_EINVAL, "H and I must be positive");
  if (!(eps >= 0.f) || eps == INFINITY) return set_error(FD_EINVAL, "eps must be a finite value >= 0");
  if (M == 0) return FD_OK;
  if (!y || !mid || !hidden || !norm_w || !w_gate_up8 || !gate_up_scale || !w_down8 || !down_scale)
    return set_error(FD_EINVAL, "null pointer argument");
  if (check_mlp_buffers(y, mid, hidden, M, H, I, 2) != FD_OK) return FD_EINVAL;
  if (H % 16 != 0 || I % 16 != 0) return set_error(FD_EUNSUPPORTED, "H and I must be multiples of 16");
  if (H > 0x7fffffffLL || 2 * I > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "too large");
  if (!aligned16(y) || !aligned16(mid) || !aligned16(hidden) || !aligned16(norm_w) ||
      !aligned16(w_gate_up8) || !aligned16(w_down8))
    return set_error(FD_EUNSUPPORTED, "operands must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint8_t* wgu = static_cast<const uint8_t*>(w_gate_up8);
  int rc;
  const bool res = act_dtype == FD_F16 ? res_takes<f16, uint8_t, 8, 3>(M, I, H, norm_w_dtype)
                                       : res_takes<bf16, uint8_t, 8, 3>(M, I, H, norm_w_dtype);
  if (res) {
    // 5-8 rows: the persistent form, the normalised rows resident in LDS and
    // only the weights streamed, eight waves with three units in flight each
    // (Llama-3-8B widths, M=8: post_attn_mlp_fp8 41.3-42.0 -> 37.7 us; four
    // waves: 41.5-43.6; the producer's row sums are not needed)
    rc = act_dtype == FD_F16 ? launch_gate_up_res<f16, uint8_t, 8, 3>(mid, hidden, wgu, gate_up_scale, (int)M,
                                                                      (int)I, (int)H, H, norm_w, norm_w_dtype,
                                                                      eps, st)
                             : launch_gate_up_res<bf16, uint8_t, 8, 3>(mid, hidden, wgu, gate_up_scale, (int)M,
                                                                       (int)I, (int)H, H, norm_w, norm_w_dtype,
                                                                       eps, st);
    if (rc != FD_OK) return rc;
  } else if (M >= kFp8MfmaMinM) {
    // the MFMA gate/up normalising inside the kernel: row sums from the producer,
    // or from a pass over x (one launch instead of the row kernel + gate/up)
    const int waves = rq && M <= 8 ? fp8_ss_waves<true, false>() : fp8_ss_waves<false, true>();
    const int units = (int)((H + kUnit - 1) / kUnit);
    const int nwv = units < waves ? units : waves;
    const size_t lds = relayout_ss_lds((int)H, waves);
    if (lds + (size_t)(waves * kWave + waves * 256) * 16 > kMaxLds)
      return set_error(FD_EUNSUPPORTED, "H too large for the norm weight's LDS stage");
    const RowSq sq = rq ? *rq : RowSq{nullptr, 0};
    const GateUpGrid gg = relayout_grid((int)I);
    auto launch = [&](auto kernel, auto* out, auto* in) {
      if (!allow_lds(kernel, lds)) return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", lds);
      hipLaunchKernelGGL(kernel, dim3(gg.blocks), dim3(nwv * kWave), lds, st, out, in, wgu, gate_up_scale, (int)M,
                         (int)H, (int)I, norm_w, norm_w_dtype, eps, sq, gg.big);
      return (int)FD_OK;
    };
    auto run = [&](auto k16, auto kb16) {
      return act_dtype == FD_F16 ? launch(k16, static_cast<f16*>(mid), static_cast<const f16*>(hidden))
                                 : launch(kb16, static_cast<bf16*>(mid), static_cast<const bf16*>(hidden));
    };
    if (gg.mix) {
      if (rq)
        rc = M <= 8 ? run(mlp_gate_up_fp8_relayout_kernel<f16, true, false, true>,
                          mlp_gate_up_fp8_relayout_kernel<bf16, true, false, true>)
                    : run(mlp_gate_up_fp8_relayout_kernel<f16, false, false, true>,
                          mlp_gate_up_fp8_relayout_kernel<bf16, false, false, true>);
      else
        rc = M <= 8 ? run(mlp_gate_up_fp8_relayout_kernel<f16, true, true, true>,
                          mlp_gate_up_fp8_relayout_kernel<bf16, true, true, true>)
                    : run(mlp_gate_up_fp8_relayout_kernel<f16, false, true, true>,
                          mlp_gate_up_fp8_relayout_kernel<bf16, false, true, true>);
    } else if (rq) {
      rc = M <= 8 ? run(mlp_gate_up_fp8_relayout_kernel<f16, true, false>,
                        mlp_gate_up_fp8_relayout_kernel<bf16, true, false>)
                  : run(mlp_gate_up_fp8_relayout_kernel<f16, false, false>,
                        mlp_gate_up_fp8_relayout_kernel<bf16, false, false>);
    } else {
      rc = M <= 8 ? run(mlp_gate_up_fp8_relayout_kernel<f16, true, true>,
                        mlp_gate_up_fp8_relayout_kernel<bf16, true, true>)
                  : run(mlp_gate_up_fp8_relayout_kernel<f16, false, true>,
                        mlp_gate_up_fp8_relayout_kernel<bf16, false, true>);
    }
    if (rc != FD_OK) return rc;
  } else if (fp8_px_takes((int)M, (int)(2 * I), (int)H)) {
    const Epi none_e{};
    const Rope none{};
    rc = act_dtype == FD_F16
             ? launch_fp8_px_m<f16, kPxGateUp>((int)M, mid, hidden, wgu, gate_up_scale, (int)(2 * I), (int)H, H, H,
                                               I, 1, none_e, norm_w, norm_w_dtype, eps, none, st)
             : launch_fp8_px_m<bf16, kPxGateUp>((int)M, mid, hidden, wgu, gate_up_scale, (int)(2 * I), (int)H, H,
                                                H, I, 1, none_e, norm_w, norm_w_dtype, eps, none, st);
    if (rc != FD_OK) return rc;
  } else {
    rc = act_dtype == FD_F16
             ? launch_mlp_fp8_m<f16>((int)M, mid, hidden, norm_w, norm_w_dtype, wgu,
                                     gate_up_scale, (int)H, (int)I, eps, st)
             : launch_mlp_fp8_m<bf16>((int)M, mid, hidden, norm_w, norm_w_dtype, wgu,
                                      gate_up_scale, (int)H, (int)I, eps, st);
    if (rc != FD_OK) return rc;
  }
  Epi e;
  e.bias = nullptr;
  e.bias_dtype = act_dtype;
  e.sb = 0;
  e.row = hidden;
  e.row_dtype = act_dtype;
  e.srm = H;
  e.srn = 1;
  e.ss = ss_out;
  const uint8_t* wd = static_cast<const uint8_t*>(w_down8);
  if (!ss_out && fp8_px_takes((int)M, (int)H, (int)I)) {
    const Rope none{};
    rc = act_dtype == FD_F16
             ? launch_fp8_px_m<f16, kPxGemv>((int)M, y, mid, wd, down_scale, (int)H, (int)I, I, I, H, 1, e, nullptr,
                                             FD_F32, 0.f, none, st)
             : launch_fp8_px_m<bf16, kPxGemv>((int)M, y, mid, wd, down_scale, (int)H, (int)I, I, I, H, 1, e,
                                              nullptr, FD_F32, 0.f, none, st);
  } else {
    rc = act_dtype == FD_F16
             ? launch_gemv_fp8_m<f16>((int)M, y, mid, wd, down_scale, (int)H, (int)I, I, I, H, 1, e, st)
             : launch_gemv_fp8_m<bf16>((int)M, y, mid, wd, down_scale, (int)H, (int)I, I, I, H, 1, e, st);
  }
  if (rc != FD_OK) return rc;
  return check_launch();
}

}  // namespace
}  // namespace fd

extern "C" int fd_post_attn_mlp_fp8(void* y, void* mid, const void* hidden, const void* norm_w,
                                    int norm_w_dtype, const void* w_gate_up8,
                                    const float* gate_up_scale, const void* w_down8,
                                    const float* down_scale, int64_t M, int64_t H, int64_t I,
                                    float eps, int act_dtype, void* stream) {
  return fd::post_attn_mlp_fp8_entry(y, mid, hidden, norm_w, norm_w_dtype, w_gate_up8, gate_up_scale, w_down8,
                                     down_scale, M, H, I, eps, act_dtype, nullptr, nullptr, stream);
}

extern "C" int fd_post_attn_mlp_fp8_sumsq(void* y, void* mid, const void* hidden, const void* norm_w,
                                          int norm_w_dtype, const void* w_gate_up8, const float* gate_up_scale,
                                          const void* w_down8, const float* down_scale, int64_t M, int64_t H,
                                          int64_t I, float eps, int act_dtype, const float* ss_in,
                                          int64_t ss_tiles, float* ss_out, void* stream) {
  using namespace fd;
  const int rc = check_sumsq(M >= kFp8MfmaMinM && M <= 16, ss_in, ss_tiles, H, ss_out);
  if (rc != FD_OK) return rc;
  const RowSq rq{ss_in, (int)ss_tiles};
  return post_attn_mlp_fp8_entry(y, mid, hidden, norm_w, norm_w_dtype, w_gate_up8, gate_up_scale, w_down8,
                                 down_scale, M, H, I, eps, act_dtype, ss_in ? &rq : nullptr, ss_out, stream);
}

namespace fd {
namespace {

int pre_attn_qkv_fp8_entry(void* y, void* normed, const void* hidden, const void* norm_w, int norm_w_dtype,
                           const void* w_qkv8, const float* w_scale, const void* bias, int bias_dtype,
                           const void* cos, const void* sin, int cs_dtype, int64_t cs_row_stride, int64_t M,
                           int64_t H, int64_t N, int64_t rope_cols, int64_t head_dim, float eps, int act_dtype,
                           const RowSq* rq, void* stream) {
  const bool mfma = M >= kFp8MfmaMinM;
  Epi e;
  Rope rp;
  bool empty = false;
  const int checked = qkv_prepare(y, normed, hidden, norm_w, norm_w_dtype, w_qkv8, bias,
                                  bias_dtype, cos, sin, cs_dtype, cs_row_stride, M, H, N,
                                  rope_cols, head_dim, eps, act_dtype, false, e, rp, empty);
  if (checked != FD_OK || empty) return checked;
  if (!w_scale) return set_error(FD_EINVAL, "null pointer argument");
  if (H % 16 != 0) return set_error(FD_EUNSUPPORTED, "the fp8 QKV needs H %% 16 == 0");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint8_t* w = static_cast<const uint8_t*>(w_qkv8);
  if (fp8_px_takes((int)M, (int)N, (int)H)) {
    const int rc = act_dtype == FD_F16
                       ? launch_fp8_px_m<f16, kPxQkv>((int)M, y, hidden, w, w_scale, (int)N, (int)H, H, H, N, 1, e,
                                                    norm_w, norm_w_dtype, eps, rp, st)
                       : launch_fp8_px_m<bf16, kPxQkv>((int)M, y, hidden, w, w_scale, (int)N, (int)H, H, H, N, 1, e,
                                                     norm_w, norm_w_dtype, eps, rp, st);
    if (rc != FD_OK) return rc;
  } else if (mfma) {  // one launch: the RMSNorm folded into the MFMA kernel
    rp.tiles = (int)(rope_cols / 16);
    FoldNorm fn{norm_w, norm_w_dtype, eps};
    if (rq) fn.sq = *rq;
    const int rc = act_dtype == FD_F16
                       ? launch_gemv_fp8_mfma<f16>((int)M, y, hidden, w, w_scale, (int)N, (int)H, H, H, N, 1,
                                                   e, st, &rp, &fn)
                       : launch_gemv_fp8_mfma<bf16>((int)M, y, hidden, w, w_scale, (int)N, (int)H, H, H, N,
                                                    1, e, st, &rp, &fn);
    if (rc != FD_OK) return rc;
  } else {
    const int rc = act_dtype == FD_F16
                       ? launch_qkv_fp8_m<f16>((int)M, y, hidden, norm_w, norm_w_dtype, w, w_scale,
                                               (int)H, (int)N, eps, e, rp, st)
                       : launch_qkv_fp8_m<bf16>((int)M, y, hidden, norm_w, norm_w_dtype, w,
                                                w_scale, (int)H, (int)N, eps, e, rp, st);
    if (rc != FD_OK) return rc;
  }
  return check_launch();
}

}  // namespace
}  // namespace fd

extern "C" int fd_pre_attn_qkv_fp8(void* y, void* normed, const void* hidden, const void* norm_w,
                                   int norm_w_dtype, const void* w_qkv8, const float* w_scale,
                                   const void* bias, int bias_dtype, const void* cos,
                                   const void* sin, int cs_dtype, int64_t cs_row_stride, int64_t M,
                                   int64_t H, int64_t N, int64_t rope_cols, int64_t head_dim,
                                   float eps, int act_dtype, void* stream) {
  return fd::pre_attn_qkv_fp8_entry(y, normed, hidden, norm_w, norm_w_dtype, w_qkv8, w_scale, bias, bias_dtype,
                                    cos, sin, cs_dtype, cs_row_stride, M, H, N, rope_cols, head_dim, eps,
                                    act_dtype, nullptr, stream);
}

extern "C" int fd_pre_attn_qkv_fp8_sumsq(void* y, const void* hidden, const void* norm_w, int norm_w_dtype,
                                         const void* w_qkv8, const float* w_scale, const void* bias,
                                         int bias_dtype, const void* cos, const void* sin, int cs_dtype,
                                         int64_t cs_row_stride, int64_t M, int64_t H, int64_t N,
                                         int64_t rope_cols, int64_t head_dim, float eps, int act_dtype,
                                         const float* ss_in, int64_t ss_tiles, void* stream) {
  using namespace fd;
  if (!ss_in) return set_error(FD_EINVAL, "null pointer argument");
  const int rc = check_sumsq(M >= kFp8MfmaMinM && M <= 16, ss_in, ss_tiles, H, nullptr);
  if (rc != FD_OK) return rc;
  const RowSq rq{ss_in, (int)ss_tiles};
  return pre_attn_qkv_fp8_entry(y, nullptr, hidden, norm_w, norm_w_dtype, w_qkv8, w_scale, bias, bias_dtype, cos,
                                sin, cs_dtype, cs_row_stride, M, H, N, rope_cols, head_dim, eps, act_dtype, &rq,
                                stream);
}
