// Shared pieces of the GEMV-family kernels (gemv.hip, fp8.hip): tile constants,
// the GEMV epilogue, the RMSNorm prologue of the fused kernels, and the host-side
// launch-shape helpers.
#pragma once

#include <atomic>

#include "fd_device.h"
#include "fd_host.h"

namespace fd {

constexpr int kMaxWaves = 8;      // waves per workgroup (512 threads)
constexpr int kChunk = 512;       // K elements one wave covers per SIMT step
constexpr int kUnit = 128;        // K elements of one MFMA unit (4 steps of 32)

// Unit i of a wave's share of an MFMA workgroup's K sweep: the wave takes units
// wave, wave + nw, ... of a sweep that starts at unit `off` and wraps, so every
// unit is taken once. Workgroups are dealt to the eight XCDs in turn, and
// blockIdx / 8 numbers a workgroup among those sharing one L2; starting each at
// its own unit keeps them from reading the same activation lines in step
// (N = 4096, K = 14336, M = 8: 20.7 against 21.7 us).
__device__ __forceinline__ int sweep_offset(int units) {
  return units > 0 ? (int)(blockIdx.x >> 3) % units : 0;
}
__device__ __forceinline__ int sweep_unit(int wave, int i, int nw, int off, int units) {
  const int u = wave + i * nw + off;  // < 2 * units: wave + i * nw < units, off < units
  return u - (u >= units ? units : 0);
}

// ---------------------------------------------------------------------------
// Global -> LDS streaming for the MFMA forms (gfx950 global_load_lds_dwordx4).
// One instruction moves 16 bytes per lane straight into LDS, lane L landing at
// byte 16*L of the (wave-uniform) destination, without passing through VGPRs,
// so a wave can keep several weight tiles in flight at the register cost of
// none. The compiler orders a DMA against later LDS reads only by waiting for
// every outstanding load (vmcnt(0)), which would drain the ring; so the ring is
// read with ds_read_b128 in inline assembly, out of its view, and each read is
// guarded by an explicit s_waitcnt vmcnt(n) that lets exactly the younger
// DMAs stay in flight (vector-memory loads complete in issue order).

__device__ __forceinline__ void dma16(const void* src, u32x4* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 0);
}
// The same with the nontemporal hint (cache policy 2: `nt`), for weight streams
// read exactly once (Llama-3-8B widths, M=8 step: down projection 23.0 -> 21.5 us,
// QKV 13.8 -> 13.3; E4M3 15.7 -> 15.3 and 11.8 -> 11.6).
__device__ __forceinline__ void dma16_nt(const void* src, u32x4* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 2);
}

// Byte address of an LDS location, as ds_read takes it.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void ds_zero16(unsigned addr) {
  const u32x4 z = {0u, 0u, 0u, 0u};
  asm volatile("ds_write_b128 %0, %1" ::"v"(addr), "v"(z) : "memory");
}

__device__ __forceinline__ void ds_write16(unsigned addr, const u32x4& v) {
  asm volatile("ds_write_b128 %0, %1" ::"v"(addr), "v"(v) : "memory");
}

__device__ __forceinline__ u32x4 ds_read16(unsigned addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}


constexpr int pow2_ceil(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Optional epilogue operands: bias[n] then row_add[m,n], added in float32 before
// the single rounding of the output (kernels.py:657-672 order).
struct Epi {
  const void* bias;
  int bias_dtype;
  int64_t sb;
  const void* row;
  int row_dtype;
  int64_t srm, srn;
  // MFMA plain tiles only: each tile t also writes ss[t*16 + m], the float32 sum
  // of its rounded outputs squared in row m (zero for m >= M), for the RMSNorm
  // of a kernel that reads this output next
  float* ss = nullptr;
};

__device__ __forceinline__ float epilogue(const Epi& e, float acc, int64_t m, int64_t n) {
  if (e.bias) acc += load_any(e.bias, e.bias_dtype, n * e.sb);
  if (e.row) acc += load_any(e.row, e.row_dtype, m * e.srm + n * e.srn);
  return acc;
}

// 8 consecutive norm-weight values of a run-time dtype (16-byte aligned).
__device__ __forceinline__ void load8_norm_w(const void* p, int dtype, int64_t k, float (&f)[8]) {
  if (dtype == FD_F32)
    load8_f32<float>(static_cast<const float*>(p) + k, f);
  else if (dtype == FD_BF16)
    load8_f32<bf16>(static_cast<const bf16*>(p) + k, f);
  else
    load8_f32<f16>(static_cast<const f16*>(p) + k, f);
}

__device__ __forceinline__ void store_norm_chunk(float* wl, const u32x4& v, int c, int dtype) {
  if (dtype == FD_F32) {
    reinterpret_cast<f32x4*>(wl)[c] = __builtin_bit_cast(f32x4, v);
    return;
  }
  float f[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t u = v[j];
    if (dtype == FD_BF16) {
      f[2 * j] = __builtin_bit_cast(float, u << 16);
      f[2 * j + 1] = __builtin_bit_cast(float, u & 0xffff0000u);
    } else {
      f[2 * j] = (float)__builtin_bit_cast(f16, (unsigned short)(u & 0xffffu));
      f[2 * j + 1] = (float)__builtin_bit_cast(f16, (unsigned short)(u >> 16));
    }
  }
  reinterpret_cast<f32x4*>(wl)[2 * c] = f32x4{f[0], f[1], f[2], f[3]};
  reinterpret_cast<f32x4*>(wl)[2 * c + 1] = f32x4{f[4], f[5], f[6], f[7]};
}

// Row sums of squares a producer kernel wrote for this kernel's input (Epi::ss
// layout: `parts` tiles of 16 floats), or p == nullptr to derive them from x.
struct RowSq {
  const float* p;
  int parts;
};

// RMSNorm folded into an MFMA kernel. The workgroup stages the norm weight in
// LDS as float32 (wl; zeros from H to `hp`, a whole number of K units) and the
// inverse RMS of every activation row (inv[m] = 1/sqrt(mean(x[m]^2) + eps),
// zero for rows past M), from the producer's row sums (rq) or from x; each B
// fragment of raw activations is then normalised as the row kernels do it,
// round(x * inv[m] * w[k]) (norm.hip).
//
// One memory round trip: a thread's first 16-byte chunks of the norm weight and
// its first producer tiles, or its first two 8-element slices of every row (one
// up to 8 rows), are all loaded before any is used (every load unconditional,
// indices clamped). `after_loads()` runs once, right after those loads are
// issued: a caller that issues its weight stream there queues it behind them,
// and since vector-memory loads complete in issue order, waiting for the
// prologue's data then never waits for the weights. NTMAX, the launch's
// largest block size, sizes that first round to 512 weight chunks and 256
// producer tiles (H up to 4096 with a 16-bit weight); wider rows take further
// rounds after after_loads(). H % 8 == 0; `scratch` holds kMaxWaves *
// pow2_ceil(MMAX) floats. Ends with a barrier (wl and inv are then visible).
// FROM_X false: only the RowSq form is compiled (rq.p must be set), which keeps
// the x passes' registers out of a kernel that never runs them. STAGE false:
// the caller reads the norm weight itself; wl is left untouched.
template <typename T, int MMAX, bool FROM_X, int NTMAX, bool STAGE = true, typename AfterLoads>
__device__ __forceinline__ void norm_prologue(float* wl, float* inv, float* scratch, const void* nwp,
                                              int nw_dtype, const T* x, int64_t sxm, int M, int H,
                                              int hp, float eps, const RowSq& rq, AfterLoads&& after_loads) {
  typedef typename Vec8<T>::type V8;
  constexpr int MP = pow2_ceil(MMAX);
  // weight chunks per thread in the first round (two where an x pass of more
  // than 8 rows holds its registers)
  constexpr int WR = NTMAX >= 256 || (FROM_X && MMAX > 8) ? 2 : 512 / NTMAX;
  constexpr int TQ = NTMAX >= 256 ? 1 : 256 / NTMAX;  // producer tiles per thread in the first round
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nt = block_threads(), nwv = nt / kWave;
  const int wchunks = H / (nw_dtype == FD_F32 ? 4 : 8);  // 16-byte chunks of the weight
  const u32x4* wsrc = static_cast<const u32x4*>(nwp);
  u32x4 wr[WR];
  if constexpr (STAGE) {
#pragma unroll
    for (int i = 0; i < WR; ++i) {
      const int c = tid + i * nt;
      wr[i] = wsrc[c < wchunks ? c : 0];
    }
  }
  auto stage_w = [&]() {
    if constexpr (STAGE) {
#pragma unroll
      for (int i = 0; i < WR; ++i) {
        const int c = tid + i * nt;
        if (c < wchunks) store_norm_chunk(wl, wr[i], c, nw_dtype);
      }
      for (int c = tid + WR * nt; c < wchunks; c += nt) store_norm_chunk(wl, wsrc[c], c, nw_dtype);
      for (int k = H + tid; k < hp; k += nt) wl[k] = 0.f;
    }
  };
  float ss[MP];
#pragma unroll
  for (int m = 0; m < MP; ++m) ss[m] = 0.f;
  bool from_sq = true;
  if constexpr (FROM_X) from_sq = rq.p != nullptr;
  if (from_sq) {
    // the producer's tile sums: thread tid adds tiles tid, tid + nt, ... (rows
    // past M are added too and discarded below)
    constexpr int MQ = (MMAX + 3) / 4;
    auto tile_rows = [&](int t, f32x4 (&q)[MQ]) {
      const f32x4* src = reinterpret_cast<const f32x4*>(rq.p + (int64_t)(t < rq.parts ? t : 0) * 16);
#pragma unroll
      for (int i = 0; i < MQ; ++i) q[i] = src[i];
    };
    auto add_tile = [&](const f32x4 (&q)[MQ]) {
#pragma unroll
      for (int m = 0; m < MMAX; ++m) ss[m] += q[m / 4][m % 4];
    };
    f32x4 q[TQ][MQ];
#pragma unroll
    for (int i = 0; i < TQ; ++i) tile_rows(tid + i * nt, q[i]);
    after_loads();
    stage_w();
#pragma unroll
    for (int i = 0; i < TQ; ++i)
      if (tid + i * nt < rq.parts) add_tile(q[i]);
    for (int t = tid + TQ * nt; t < rq.parts; t += nt) {
      tile_rows(t, q[0]);
      add_tile(q[0]);
    }
  } else if constexpr (FROM_X) {
    const int k0 = tid * 8, k1 = k0 + nt * 8;
    V8 h[MMAX], h1[MMAX <= 8 ? MMAX : 1];
#pragma unroll
    for (int m = 0; m < MMAX; ++m) h[m] = load8<T>(x + (m < M ? m : M - 1) * sxm + (k0 < H ? k0 : 0));
    if constexpr (MMAX <= 8) {  // the second pass's loads in the same round trip
#pragma unroll
      for (int m = 0; m < MMAX; ++m) h1[m] = load8<T>(x + (m < M ? m : M - 1) * sxm + (k1 < H ? k1 : 0));
    }
    after_loads();
    stage_w();
    // x^2 two at a time with v_dot2_f32_f16 / _bf16 (no conversions); a slice past
    // H keeps the old sums, and rows past M get inv = 0 whatever they summed
    auto add = [&](int k) {
#pragma unroll
      for (int m = 0; m < MMAX; ++m) {
        const u32x4 p = __builtin_bit_cast(u32x4, h[m]);
        float s = ss[m];
#pragma unroll
        for (int j = 0; j < 4; ++j) s = sq_dot2<T>(p[j], s);
        ss[m] = k < H ? s : ss[m];
      }
    };
    add(k0);
    int k = k1;
    if constexpr (MMAX <= 8) {
#pragma unroll
      for (int m = 0; m < MMAX; ++m) h[m] = h1[m];
      add(k1);
      k += nt * 8;
    }
    for (; k < H; k += nt * 8) {
#pragma unroll
      for (int m = 0; m < MMAX; ++m) h[m] = load8<T>(x + (m < M ? m : M - 1) * sxm + k);
      add(k);
    }
  }
  butterfly_sum<MP>(ss, lane);
  if (butterfly_writer<MP>(lane)) scratch[wave * MP + butterfly_index<MP>(lane)] = ss[0];
  __syncthreads();
  if (tid < MMAX) {
    float s = 0.f;
    for (int i = 0; i < nwv; ++i) s += scratch[i * MP + tid];
    inv[tid] = tid < M ? rsqrtf(s / (float)H + eps) : 0.f;
  }
  __syncthreads();
}

// x * inv in float32 for the low / high f16 of a packed pair: one v_fma_mix_f32
// (f16 operand converted exactly, addend -0.0, so the result is the rounded
// product, sign of zero included) in place of a conversion and a multiply.
// The compiler folds fma(x, inv, -0) back into a multiply, hence the asm.
__device__ __forceinline__ float mul_lo_f16(unsigned pair, float inv) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(inv));
  return r;
}
__device__ __forceinline__ float mul_hi_f16(unsigned pair, float inv) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(inv));
  return r;
}

// B fragment of raw activations -> round(x * inv * w) for its 8 k (w as 8 floats).
template <typename T>
__device__ __forceinline__ u32x4 norm_frag(const u32x4& raw, float inv, const u32x4& w0, const u32x4& w1) {
  if constexpr (std::is_same<T, f16>::value) {
    const f32x4 wa = __builtin_bit_cast(f32x4, w0), wb = __builtin_bit_cast(f32x4, w1);
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      o[2 * j] = (f16)(mul_lo_f16(raw[j], inv) * wa[2 * j]);
      o[2 * j + 1] = (f16)(mul_hi_f16(raw[j], inv) * wa[2 * j + 1]);
      o[2 * j + 4] = (f16)(mul_lo_f16(raw[j + 2], inv) * wb[2 * j]);
      o[2 * j + 5] = (f16)(mul_hi_f16(raw[j + 2], inv) * wb[2 * j + 1]);
    }
    return __builtin_bit_cast(u32x4, o);
  }
  typedef typename Vec8<T>::type V8;
  const V8 h = __builtin_bit_cast(V8, raw);
  const f32x4 wa = __builtin_bit_cast(f32x4, w0), wb = __builtin_bit_cast(f32x4, w1);
  V8 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[i] = from_f32<T>(to_f32(h[i]) * inv * wa[i]);
    o[i + 4] = from_f32<T>(to_f32(h[i + 4]) * inv * wb[i]);
  }
  return __builtin_bit_cast(u32x4, o);
}

// a * w in float32 for the low / high f16 of the packed pair `w`: the same
// v_fma_mix_f32 form (the f16 converted exactly, the product rounded once).
__device__ __forceinline__ float mul_f32_lo_f16(float a, unsigned w) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(w));
  return r;
}
__device__ __forceinline__ float mul_f32_hi_f16(float a, unsigned w) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(w));
  return r;
}

// norm_frag with the 8 norm weights in T (`wt`, exact in float32): the same
// float32 products, so the same rounded results.
template <typename T>
__device__ __forceinline__ u32x4 norm_frag_w(const u32x4& raw, float inv, const u32x4& wt) {
  if constexpr (std::is_same<T, f16>::value) {
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[2 * j] = (f16)mul_f32_lo_f16(mul_lo_f16(raw[j], inv), wt[j]);
      o[2 * j + 1] = (f16)mul_f32_hi_f16(mul_hi_f16(raw[j], inv), wt[j]);
    }
    return __builtin_bit_cast(u32x4, o);
  }
  typedef typename Vec8<T>::type V8;
  const V8 h = __builtin_bit_cast(V8, raw), wv = __builtin_bit_cast(V8, wt);
  V8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(to_f32(h[i]) * inv * to_f32(wv[i]));
  return __builtin_bit_cast(u32x4, o);
}

// LDS row stride of the staged activations: H plus 16 bytes, so the 16 rows an
// MFMA B operand reads at one k land in different LDS banks.
__host__ __device__ __forceinline__ int xs_stride(int H) { return H + 8; }

// Stage round(hidden * rsqrt(mean(hidden^2) + eps) * norm_w) for all M rows in
// LDS (xs, [M][xs_stride(H)]). `scratch` needs kMaxWaves*16 + 16 floats.
template <typename T, int MMAX>
__device__ __forceinline__ void stage_normed(T* xs, float* scratch, const T* hidden,
                                             const void* nwp, int nw_dtype, int M, int H,
                                             float eps) {
  const int XS = xs_stride(H);
  typedef typename Vec8<T>::type V8;
  constexpr int MP = pow2_ceil(MMAX);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nt = block_threads(), nwv = nt / kWave;
  float ss[MP];
#pragma unroll
  for (int m = 0; m < MP; ++m) ss[m] = 0.f;
  for (int k = tid * 8; k < H; k += nt * 8) {
#pragma unroll
    for (int m = 0; m < MMAX; ++m) {
      if (m < M) {
        V8 h = load8<T>(hidden + (int64_t)m * H + k);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss[m] += to_f32(h[i]) * to_f32(h[i]);
      }
    }
  }
  butterfly_sum<MP>(ss, lane);
  float* inv = scratch + kMaxWaves * MP;
  if (butterfly_writer<MP>(lane)) scratch[wave * MP + butterfly_index<MP>(lane)] = ss[0];
  __syncthreads();
  if (tid < M) {
    float s = 0.f;
    for (int i = 0; i < nwv; ++i) s += scratch[i * MP + tid];
    inv[tid] = rsqrtf(s / (float)H + eps);
  }
  __syncthreads();
  for (int k = tid * 8; k < H; k += nt * 8) {
    float wf[8];
    load8_norm_w(nwp, nw_dtype, k, wf);
#pragma unroll
    for (int m = 0; m < MMAX; ++m) {
      if (m < M) {
        V8 h = load8<T>(hidden + (int64_t)m * H + k);
        const float s = inv[m];
        V8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(to_f32(h[i]) * s * wf[i]);
        store8<T>(xs + (int64_t)m * XS + k, o);
      }
    }
  }
  __syncthreads();
}

// Register form of the same prologue for small M, split so the weight stream
// can start in between: norm_load issues every global load the norm needs
// (this thread's KIT 8-element slices of each hidden row and the raw bytes of
// the norm weight) before the caller issues its first weight loads, and
// norm_store reduces, converts, rounds and stages in LDS from registers. Every
// load is unconditional (slices past H and rows past M read an in-bounds
// address and are masked later): a load under a branch leaves the compiler
// unsure how many loads are outstanding, and it then waits for all of them,
// the weight loads included, before the norm's first use. Usable when
// H <= KIT * block_threads() * 8 (norm_in_regs); the same summation order and
// rounding as stage_normed.
template <typename T, int MMAX, int KIT>
struct NormRegs {
  typename Vec8<T>::type h[KIT][MMAX];
  u32x4 w0[KIT], w1[KIT];  // 8 norm-weight values: 16 bytes (fp16/bf16) or 32 (fp32)
};

template <typename T, int MMAX, int KIT>
__device__ __forceinline__ void norm_load(NormRegs<T, MMAX, KIT>& c, const T* hidden,
                                          const void* nwp, int nw_dtype, int M, int H) {
  const bool is32 = nw_dtype == FD_F32;
  const int esz = is32 ? 4 : 2;
#pragma unroll
  for (int it = 0; it < KIT; ++it) {
    const int k = (threadIdx.x + it * block_threads()) * 8;
    const int kc = k < H ? k : 0;
#pragma unroll
    for (int m = 0; m < MMAX; ++m)
      c.h[it][m] = load8<T>(hidden + (int64_t)(m < M ? m : 0) * H + kc);
    const char* pb = static_cast<const char*>(nwp) + (int64_t)kc * esz;
    c.w0[it] = *reinterpret_cast<const u32x4*>(pb);
    c.w1[it] = *reinterpret_cast<const u32x4*>(pb + (is32 ? 16 : 0));
  }
}

// The 8 float32 norm-weight values of a norm_load slice.
__device__ __forceinline__ void norm_w8(const u32x4& w0, const u32x4& w1, int dtype,
                                        float (&f)[8]) {
  if (dtype == FD_F32) {
    const f32x4 a = __builtin_bit_cast(f32x4, w0), b = __builtin_bit_cast(f32x4, w1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = a[i];
      f[i + 4] = b[i];
    }
  } else if (dtype == FD_BF16) {
    const bf16x8 a = __builtin_bit_cast(bf16x8, w0);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = to_f32(a[i]);
  } else {
    const f16x8 a = __builtin_bit_cast(f16x8, w0);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = to_f32(a[i]);
  }
}

template <typename T, int MMAX, int KIT>
__device__ __forceinline__ void norm_store(const NormRegs<T, MMAX, KIT>& c, T* xs,
                                           float* scratch, int nw_dtype, int M, int H,
                                           float eps) {
  const int XS = xs_stride(H);
  typedef typename Vec8<T>::type V8;
  constexpr int MP = pow2_ceil(MMAX);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nwv = block_threads() / kWave;
  float ss[MP];
#pragma unroll
  for (int m = 0; m < MP; ++m) ss[m] = 0.f;
#pragma unroll
  for (int it = 0; it < KIT; ++it) {
    const bool in = (tid + it * block_threads()) * 8 < H;
#pragma unroll
    for (int m = 0; m < MMAX; ++m) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = in && m < M ? to_f32(c.h[it][m][i]) : 0.f;
        ss[m] += v * v;
      }
    }
  }
  butterfly_sum<MP>(ss, lane);
  float* inv = scratch + kMaxWaves * MP;
  if (butterfly_writer<MP>(lane)) scratch[wave * MP + butterfly_index<MP>(lane)] = ss[0];
  __syncthreads();
  if (tid < M) {
    float s = 0.f;
    for (int i = 0; i < nwv; ++i) s += scratch[i * MP + tid];
    inv[tid] = rsqrtf(s / (float)H + eps);
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < KIT; ++it) {
    const int k = (tid + it * block_threads()) * 8;
    if (k < H) {
      float wf[8];
      norm_w8(c.w0[it], c.w1[it], nw_dtype, wf);
#pragma unroll
      for (int m = 0; m < MMAX; ++m) {
        if (m < M) {
          const float s = inv[m];
          V8 o;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(to_f32(c.h[it][m][i]) * s * wf[i]);
          store8<T>(xs + (int64_t)m * XS + k, o);
        }
      }
    }
  }
  __syncthreads();
}

// The K steps a persistent workgroup streams: its tiles blockIdx.x,
// blockIdx.x + gridDim.x, ... below `tiles`, each `steps` steps of `step`
// elements, flattened to s = 0 .. total-1 (this thread's slice of step s starts
// at k(s)).
struct StepPlan {
  int steps, step, kbase, total;
  __device__ __forceinline__ StepPlan(int tiles, int H, int step_, int kbase_)
      : steps((H + step_ - 1) / step_), step(step_), kbase(kbase_) {
    const int g = (int)gridDim.x;
    total = (tiles - (int)blockIdx.x + g - 1) / g * steps;
  }
  __device__ __forceinline__ int tile(int s) const { return (int)blockIdx.x + s / steps * (int)gridDim.x; }
  __device__ __forceinline__ int k(int s) const { return kbase + s % steps * step; }
  __device__ __forceinline__ bool last(int s) const { return s % steps == steps - 1; }
  // Parity of step s's tile among this workgroup's tiles.
  __device__ __forceinline__ int half(int s) const { return (s / steps) & 1; }
};

// Streams the plan's steps through two register buffers: the loads of step s+1
// are in flight while step s is consumed (and its tile's epilogue runs).
// issue(buf, s) loads step s (s < total) with every load unconditional -- lanes
// or rows out of range read an in-bounds dummy address -- so that waiting for
// one buffer never waits for the other; consume(buf, s) does the math of step s.
// The caller issues step 0 into `a` first, so a prologue can overlap it. The
// last one or two steps are peeled so no step past the plan is ever loaded.
template <typename Buf, typename Issue, typename Consume>
__device__ __forceinline__ void stream_steps(int total, Buf& a, Buf& b, Issue&& issue,
                                             Consume&& consume) {
  int s = 0;
  for (; s + 2 < total; s += 2) {
    issue(b, s + 1);
    consume(a, s);
    issue(a, s + 2);
    consume(b, s + 1);
  }
  if (s + 1 < total) {
    issue(b, s + 1);
    consume(a, s);
    consume(b, s + 1);
  } else if (s < total) {
    consume(a, s);
  }
}

// stream_steps for a caller that issued both step 0 (into `a`) and step 1 (into
// `b`, when total > 1) before a prologue, so the prologue overlaps two steps'
// loads. Same two buffers, same order of loads and math after that.
template <typename Buf, typename Issue, typename Consume>
__device__ __forceinline__ void stream_steps_issued2(int total, Buf& a, Buf& b, Issue&& issue,
                                                     Consume&& consume) {
  int s = 0;
  for (; s + 3 < total; s += 2) {
    consume(a, s);
    issue(a, s + 2);
    consume(b, s + 1);
    issue(b, s + 3);
  }
  const int left = total - s;
  if (left == 3) {
    consume(a, s);
    issue(a, s + 2);
    consume(b, s + 1);
    consume(a, s + 2);
  } else if (left == 2) {
    consume(a, s);
    consume(b, s + 1);
  } else if (left == 1) {
    consume(a, s);
  }
}

// Half-B form of the relayout kernels' activation fragments, for M <= 8 (MFMA
// columns 8-15 are padding): a lane of row r < 8 loads fragment 2p of x row r,
// a lane of row r >= 8 fragment 2p+1 of x row 15-r (half_b_row), and after any
// per-lane transform mirror16 (DPP row_mirror: lane r <-> 15-r, k group kept)
// hands each low lane its partner's fragment. Two loads and two transforms per
// unit then give the four B fragments lanes 0-7 need.
__device__ __forceinline__ int half_b_row(int r) { return r < 8 ? r : 15 - r; }

template <typename T>
__device__ __forceinline__ void load_b_half(typename Vec8<T>::type (&b)[4], const T* xh, int u, int g, int hi,
                                            int K) {
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int kb = u * kUnit + ((2 * p + hi) * 4 + g) * 8;
    b[p] = load8<T>(xh + (kb < K ? kb : 0));
  }
}

__device__ __forceinline__ u32x4 mirror16(const u32x4& v) {
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (unsigned)__builtin_amdgcn_mov_dpp((int)v[i], XlaneDpp<8>::ctrl, 0xf, 0xf, false);
  return o;
}

// B fragment s2 of MFMA unit u for lane group g (x[m][k .. k+8), k = u*128 +
// (4*s2 + g)*8), zeroed past K; the MFMA forms load it unconditionally.
__device__ __forceinline__ f16x8 unit_b(const f16x8& b, int u, int s2, int g, int K) {
  return u * kUnit + (s2 * 4 + g) * 8 < K ? b : f16x8{};
}
__device__ __forceinline__ bf16x8 unit_b(const bf16x8& b, int u, int s2, int g, int K) {
  return u * kUnit + (s2 * 4 + g) * 8 < K ? b : bf16x8{};
}

// The register prologue holds 2 slices of 8 per row and thread (H up to 16
// values per thread) and is used up to 2 rows; beyond that its registers would
// cost the weight loop occupancy, and the loop's longer math hides the prologue.
// The host decides with norm_in_regs and launches the kernel's REGS form.
constexpr int kNormRegMaxM = 2;
constexpr int kNormRegRows(int m) { return m <= kNormRegMaxM ? 2 : 1; }
__host__ __device__ __forceinline__ bool norm_in_regs(int M, int H, int threads) {
  return M <= kNormRegMaxM && H <= kNormRegRows(M) * threads * 8;
}

template <typename T>
__device__ __forceinline__ T swiglu_out(float g, float u) {
  return from_f32<T>(silu_stable(round_as<T>(g)) * round_as<T>(u));
}

constexpr int kNormScratch = kMaxWaves * 16 + 16;

// Relayout gate/up kernels that normalise from a producer's row sums (SS): at
// most this many waves, and their dynamic LDS for H columns (the norm weight
// as float32 in whole K units, inv[16], and the reduction scratch of `waves`).
constexpr int kSsWaves = 4;
__host__ __device__ constexpr size_t relayout_ss_lds(int H, int waves) {
  return ((size_t)(H + kUnit - 1) / kUnit * kUnit + 16 + (size_t)waves * 16) * sizeof(float);
}

constexpr bool kNtWeights = true;           // nontemporal weight loads (measured +10-20%)
constexpr size_t kMaxLds = 160 * 1024;       // LDS per CU on gfx950

// RoPE in the epilogue of a QKV projection (rotate-half, as the standalone
// rope op): output columns below `cols` form heads of `dim` columns; column d of
// a head pairs with d + dim/2. cos/sin row m sits at m * rs (rs = 0: one row for
// every m), in `dtype`. `tiles` tiles of S rows cover the rotated columns.
struct Rope {
  const void* cos;
  const void* sin;
  int dtype;
  int64_t rs;
  int cols;
  int dim;
  int tiles;
};

// Row placement of a tile of S weight rows. A rotated tile holds S/2 adjacent
// pairs of one head, slot s < S/2 at column q + s and slot s + S/2 at its
// partner q + s + dim/2, so both halves of every pair end in one workgroup
// (needs dim/2 % (S/2) == 0). Tiles past the rotated ones hold S consecutive rows.
template <int S>
struct TileRows {
  int64_t base;  // first row of the head (rotated) or of the tile
  int q;         // head column of slot 0 (rotated tiles)
  int hh;        // dim/2, 0 for unrotated tiles
  __device__ __forceinline__ TileRows(const Rope& rp, int tile) {
    if (tile < rp.tiles) {
      hh = rp.dim >> 1;
      const int pp = tile * (S / 2);
      const int b = pp / hh;
      q = pp - b * hh;
      base = (int64_t)b * rp.dim;
    } else {
      hh = 0;
      q = 0;
      base = (int64_t)rp.cols + (int64_t)(tile - rp.tiles) * S;
    }
  }
  __device__ __forceinline__ bool rotated() const { return hh != 0; }
  // head column of slot s (rotated tiles)
  __device__ __forceinline__ int col(int s) const { return q + s % (S / 2) + (s / (S / 2)) * hh; }
  __device__ __forceinline__ int64_t row(int s) const { return rotated() ? base + col(s) : base + s; }
};


// Table loads without a branch on the table's dtype: the raw bits of element
// i as two halfword loads (the same halfword twice for fp16/bf16, both halves
// of a float32), combined and converted only where the value is used. A dtype
// switch around the loads makes the compiler wait for each load where it
// converts it.
struct TableBits {
  uint32_t lo, hi;
};
__device__ __forceinline__ TableBits load_table_bits(const void* p, int dtype, int64_t i) {
  const unsigned short* h = static_cast<const unsigned short*>(p);
  const int64_t lo = dtype == FD_F32 ? 2 * i : i;
  const int64_t hi = dtype == FD_F32 ? 2 * i + 1 : i;
  return TableBits{h[lo], h[hi]};
}
__device__ __forceinline__ float table_value(TableBits b, int dtype) {
  if (dtype == FD_F32) return __builtin_bit_cast(float, b.lo | (b.hi << 16));
  if (dtype == FD_BF16) return __builtin_bit_cast(float, b.lo << 16);
  return (float)__builtin_bit_cast(f16, (unsigned short)b.lo);
}

// The cos/sin of a rotated 16-row MFMA tile, staged in LDS once per workgroup:
// value v = (t * rows + r) * 16 + j is table t (0 cos, 1 sin) at row r (rows =
// 1 when every token shares one table row, else M) and the tile's slot j
// (TileRows<16>::col(j): slots 8-15 are the partners dim/2 further on). A
// workgroup loads its values before its main loop, PER per thread, so they wait
// under it, and stores them to LDS before its epilogue barrier. The loads are
// unconditional: a thread without a value (or any thread of an unrotated
// tile) reads `own`, an address of its own that the kernel reads anyway.
// Loads under a branch get their registers merged at its end, which waits for
// them; and every lane of every wave reading the table itself queued the whole
// launch on the same few L2 lines (together 1.9 us of 16.4 in the fused QKV at
// M = 8).
constexpr int kTileAngles = 2 * 16 * 16;  // cos and sin, 16 slots, up to 16 rows
template <int PER>
struct AngleLoads {
  TableBits b[PER];
};
template <int PER>
__device__ __forceinline__ AngleLoads<PER> angle_loads(const Rope& rp, const TileRows<16>& tr, int M,
                                                       const void* own) {
  AngleLoads<PER> a;
  const int rows = rp.rs == 0 ? 1 : M;
  const int nt = block_threads();
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int v = (int)threadIdx.x + p * nt;
    const bool use = tr.rotated() && v < 32 * rows;
    const int t = v / (16 * rows), r = (v / 16) % rows, j = v % 16;
    const void* base = use ? (t ? rp.sin : rp.cos) : own;
    a.b[p] = load_table_bits(base, rp.dtype, use ? (int64_t)r * rp.rs + tr.col(j) : 0);
  }
  return a;
}
template <int PER>
__device__ __forceinline__ void angle_store(float* lds, const AngleLoads<PER>& a, const Rope& rp,
                                            const TileRows<16>& tr, int M) {
  const int rows = rp.rs == 0 ? 1 : M;
  const int nt = block_threads();
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int v = (int)threadIdx.x + p * nt;
    if (tr.rotated() && v < 32 * rows) lds[v] = table_value(a.b[p], rp.dtype);
  }
}

// Rotate one pair in float32 from the rounded projection outputs x1 (first
// half, head column d) and x2 (second half, column d + dim/2), as the rope op;
// the four table loads are issued before any is converted (load_table_bits).
__device__ __forceinline__ void rope_pair(const Rope& rp, int64_t m, int d, float x1, float x2,
                                          float& o1, float& o2) {
  const int64_t c = m * rp.rs + d, h = rp.dim >> 1;
  const TableBits c1 = load_table_bits(rp.cos, rp.dtype, c), s1 = load_table_bits(rp.sin, rp.dtype, c);
  const TableBits c2 = load_table_bits(rp.cos, rp.dtype, c + h), s2 = load_table_bits(rp.sin, rp.dtype, c + h);
  o1 = x1 * table_value(c1, rp.dtype) - x2 * table_value(s1, rp.dtype);
  o2 = x2 * table_value(c2, rp.dtype) + x1 * table_value(s2, rp.dtype);
}

// Per-row factor applied to a GEMV sum before the epilogue: none for fp16/bf16
// weights, the channel scale scale[n] for E4M3 codes.
struct NoScale {
  __device__ __forceinline__ float operator()(float s, int64_t) const { return s; }
};
struct RowScale {
  const float* scale;
  __device__ __forceinline__ float operator()(float s, int64_t n) const { return s * scale[n]; }
};

// The epilogue operands of a plain 16-row MFMA tile for one lane of the wave
// that writes it (lane l: column m = l%16, rows nb..nb+3 with nb = 4*(l/16)):
// bias, row_add and (E4M3) channel scale, loaded before the main loop so their
// latency hides under it instead of adding to every workgroup's end. Loads are
// unconditional and branch-free (halfword pairs, see load_table_bits): absent
// operands and out-of-range lanes read the start of `own`, an address of the
// lane's own that the kernel reads anyway (one shared address would queue every
// lane of the launch on one L2 line).
struct TileEpi {
  TableBits b[4], r[4];
  float ws[4];
};
template <bool F8>
__device__ __forceinline__ TileEpi tile_epi_loads(const Epi& e, const float* wscale, const void* own, int lane,
                                                  int64_t n0, int M, int N) {
  const int m = lane & 15, nb = (lane >> 4) * 4;
  const void* bp = e.bias ? e.bias : own;
  const void* rp = e.row ? e.row : own;
  const int bdt = e.bias ? e.bias_dtype : FD_F16, rdt = e.row ? e.row_dtype : FD_F16;
  TileEpi t;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t n = n0 + nb + i;
    const bool in = n < N, mn = in && m < M;
    t.b[i] = load_table_bits(bp, bdt, e.bias && in ? n * e.sb : 0);
    t.r[i] = load_table_bits(rp, rdt, e.row && mn ? m * e.srm + n * e.srn : 0);
    if constexpr (F8) t.ws[i] = wscale[in ? n : 0];
  }
  return t;
}

// Plain tile output from the early-loaded operands: bias, then row_add, then
// one rounding (the order of `epilogue`); with Epi::ss also the tile's row sums
// of the squared rounded outputs.
template <typename T, bool F8>
__device__ __forceinline__ void mfma_tile_out_plain(T* y, const f32x4& s, int lane, int64_t n0, const Epi& e,
                                                    const TileEpi& t, int M, int N, int64_t sym, int64_t syn) {
  const int m = lane & 15;
  const int nb = (lane >> 4) * 4;
  float q = 0.f;
  if (m < M) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = n0 + nb + i;
      if (n < N) {
        float acc = F8 ? s[i] * t.ws[i] : s[i];
        if (e.bias) acc += table_value(t.b[i], e.bias_dtype);
        if (e.row) acc += table_value(t.r[i], e.row_dtype);
        const T o = from_f32<T>(acc);
        y[m * sym + n * syn] = o;
        if (e.ss) q += to_f32(o) * to_f32(o);
      }
    }
  }
  if (e.ss) {  // lanes m, m+16, m+32, m+48 hold row m's four column groups
    q = xlane_sum<32>(q);
    q = xlane_sum<16>(q);
    if (lane < 16) e.ss[(n0 >> 4) * 16 + lane] = q;
  }
}

// Output of one 16-row MFMA tile, from the 64 lanes of one wave holding the
// cross-wave sums: lane l has rows nb..nb+3 (nb = 4*(l/16)) of column m = l%16.
// With ROPE the rows follow TileRows<16>, and a rotated tile rotates its rounded
// outputs: lanes 0-31 hold slots 0-7 and lanes 32-63 their partners 8-15 (same
// m), one lane-xor-32 exchange apart, so every lane of the wave must call this;
// `ang` is the tile's staged cos/sin (angle_store) and `ang_rs` the table's row
// stride (0: one row for every m); read in rotated tiles only.
template <typename T, bool ROPE, typename Scale>
__device__ __forceinline__ void mfma_tile_out(T* y, const f32x4& s, int lane, int64_t n0,
                                              const TileRows<16>& tr, const Epi& e,
                                              const float* ang, int64_t ang_rs, const Scale& sc,
                                              int M, int N, int64_t sym, int64_t syn) {
  const int m = lane & 15;
  const int nb = (lane >> 4) * 4;
  if (ROPE && tr.rotated()) {
    float v[4], pv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = tr.row(nb + i);
      v[i] = m < M ? round_as<T>(epilogue(e, sc(s[i], n), m, n)) : 0.f;
      pv[i] = xlane_partner32(v[i], lane);
    }
    if (m < M) {
      const bool first = nb < 8;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // the rope op's pair rotation: x1 cos - x2 sin (first half), x2 cos + x1 sin
        const float x1 = first ? v[i] : pv[i], x2 = first ? pv[i] : v[i];
        const int rows = ang_rs == 0 ? 1 : M, r = ang_rs == 0 ? 0 : m;
        const float c = ang[r * 16 + nb + i], sn = ang[(rows + r) * 16 + nb + i];
        const float o = first ? x1 * c - x2 * sn : x2 * c + x1 * sn;
        y[m * sym + tr.row(nb + i) * syn] = from_f32<T>(o);
      }
    }
  } else if (m < M) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = ROPE ? tr.row(nb + i) : n0 + nb + i;
      if (n < N) y[m * sym + n * syn] = from_f32<T>(epilogue(e, sc(s[i], n), m, n));
    }
  }
}

// Output of one fused-QKV SIMT tile of R rows placed by TileRows<R>, from the
// waves' partial sums (wave i, slot r*M + m at part[i*V + r*M + m]): bias,
// rounding, and in rotated tiles the rotation of pairs (slot p, slot p + R/2).
template <typename T, int M, int R, typename Scale>
__device__ __forceinline__ void qkv_tile_out(T* y, const float* part, int V, int nw,
                                             const TileRows<R>& tr, const Epi& e, const Rope& rp,
                                             const Scale& sc, int N) {
  constexpr int P = R / 2;
  if (tr.rotated()) {
    for (int t = threadIdx.x; t < P * M; t += block_threads()) {
      const int p = t / M, m = t % M;
      float s1 = 0.f, s2 = 0.f;
      for (int i = 0; i < nw; ++i) {
        s1 += part[i * V + p * M + m];
        s2 += part[i * V + (p + P) * M + m];
      }
      const int64_t n1 = tr.row(p), n2 = tr.row(p + P);
      float o1, o2;
      rope_pair(rp, m, tr.col(p), round_as<T>(epilogue(e, sc(s1, n1), m, n1)),
                round_as<T>(epilogue(e, sc(s2, n2), m, n2)), o1, o2);
      y[m * (int64_t)N + n1] = from_f32<T>(o1);
      y[m * (int64_t)N + n2] = from_f32<T>(o2);
    }
  } else {
    for (int t = threadIdx.x; t < R * M; t += block_threads()) {
      const int r = t / M, m = t % M;
      const int64_t n = tr.row(r);
      if (n < N) {
        float s = 0.f;
        for (int i = 0; i < nw; ++i) s += part[i * V + t];
        y[m * (int64_t)N + n] = from_f32<T>(epilogue(e, sc(s, n), m, n));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side launch-shape helpers

// Waves per workgroup: one per work item (512-element chunk for SIMT, 128-element
// unit for MFMA) up to eight. An uneven split (K = 14336: 28 chunks over 8 waves)
// measured faster than an even one with fewer waves (7): more loads in flight.
inline int pick_waves(int64_t items) {
  if (items < 1) return 1;
  return items < kMaxWaves ? (int)items : kMaxWaves;
}

// The dynamic-LDS limit of a kernel must be raised before a launch above 64 KiB.
template <typename F>
inline bool allow_lds(F kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return true;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)bytes) == hipSuccess;
}

// Compute units of the current device (cached per device; host threads may race
// to fill an entry, and all of them store the same value).
inline int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (!cus) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

// Dynamic LDS of a fused kernel: the staged activations and the reduction scratch.
// LDS of the persistent fused kernels: the staged rows, then two halves of
// V * kMaxWaves partial sums (consecutive tiles alternate), which the norm
// prologue uses as scratch before the first tile.
inline size_t fused_lds(int M, int H, size_t elem, int V) {
  const int part = 2 * V * kMaxWaves;
  return (size_t)M * xs_stride(H) * elem +
         sizeof(float) * (size_t)(part > kNormScratch ? part : kNormScratch);
}

// Workgroups of the fused kernel: each stages the normalised activations in LDS
// once and then loops over weight tiles, so the grid is what can be resident at
// once, at most `per_cu` per CU and fewer when the LDS stage is large; more would
// restage x for nothing (measured at H=4096: one 8-wave workgroup per CU for the
// fp16 gate/up, two 4-wave ones for the fp8 gate/up).
inline int fused_grid(int tiles, size_t lds, int per_cu) {
  const int fit = (int)(kMaxLds / (lds ? lds : 1));
  const int cap = device_cus() * (fit < 1 ? 1 : fit < per_cu ? fit : per_cu);
  const int per = (tiles + cap - 1) / cap;
  return (tiles + per - 1) / per;
}

// Workgroups of the relayout gate/up: tiles of 16 gate + 16 up rows, and where
// their count is past a whole number of rounds over the CUs, the rows past the
// last whole round as tiles of 8 + 8 (MIX), so every CU streams about the same
// rows. At Llama-3-8B widths (I = 14336) 896 tiles of 16 + 16 put four on half
// the CUs and three on the rest (timed alone at M = 8, H = 4096: 5.61 TB/s,
// against 6.04-6.07 where they divide evenly, I = 12288 and 16384); 768 of
// them and 256 of 8 + 8 put the same rows on every CU. Tiles of 8 + 8
// throughout were slower: each activation fragment feeds half the MFMAs. The
// mix is taken only where it lowers the busiest CU's rows (in 16-row tiles:
// rounds of big tiles plus half a tile per round of small ones), e.g. not at
// I = 11008, whose leftover would put two small tiles on some CUs.
struct GateUpGrid {
  unsigned blocks;
  int big;   // workgroups with 16 + 16 rows
  bool mix;  // the rest with 8 + 8
};
inline GateUpGrid relayout_grid(int I) {
  const int cus = device_cus();
  const int t16 = (I + 15) / 16;
  const GateUpGrid plain{(unsigned)t16, t16, false};
  if (t16 <= cus || t16 % cus == 0) return plain;
  const int big = t16 - t16 % cus;
  const int small = (I - big * 16 + 7) / 8;
  const int rounds16 = (t16 + cus - 1) / cus;                 // busiest CU, plain grid
  const int halves = 2 * (big / cus) + (small + cus - 1) / cus;  // busiest CU, mixed, in 8 + 8 tiles
  if (halves >= 2 * rounds16) return plain;
  return {(unsigned)(big + small), big, true};
}

// Argument checks and operand set-up shared by the fused QKV entry points
// (fp16/bf16 and fp8 weights). `mfma`: the launch runs the RMSNorm as a row
// kernel into `normed`. Sets `empty` (and returns FD_OK) for M = 0.
inline int qkv_prepare(const void* y, const void* normed, const void* hidden, const void* norm_w,
                       int norm_w_dtype, const void* w, const void* bias, int bias_dtype,
                       const void* cos, const void* sin, int cs_dtype, int64_t cs_row_stride,
                       int64_t M, int64_t H, int64_t N, int64_t rope_cols, int64_t head_dim,
                       float eps, int act_dtype, bool mfma, Epi& e, Rope& rp, bool& empty) {
  empty = false;
  if (!check_act_dtype(act_dtype) || !check_any_dtype(norm_w_dtype, "norm_w_dtype"))
    return FD_EINVAL;
  if (M < 0 || M > 16) return set_error(FD_EINVAL, "M must be in [0, 16]");
  if (H <= 0 || N <= 0) return set_error(FD_EINVAL, "H and N must be positive");
  if (!(eps >= 0.f) || eps == INFINITY) return set_error(FD_EINVAL, "eps must be a finite value >= 0");
  if (rope_cols < 0 || rope_cols > N) return set_error(FD_EINVAL, "rope_cols must be in [0, N]");
  if (rope_cols > 0) {
    if (head_dim <= 0 || head_dim % 2 != 0) return set_error(FD_EINVAL, "head_dim must be even");
    if (rope_cols % head_dim != 0)
      return set_error(FD_EINVAL, "rope_cols must be a multiple of head_dim");
    if (!check_any_dtype(cs_dtype, "cs_dtype")) return FD_EINVAL;
    if (cs_row_stride < 0) return set_error(FD_EINVAL, "cs_row_stride must be >= 0");
    if (head_dim % 16 != 0 || head_dim > 0x7fffffffLL)
      return set_error(FD_EUNSUPPORTED, "head_dim must be a multiple of 16");
  }
  if (bias && !check_any_dtype(bias_dtype, "bias_dtype")) return FD_EINVAL;
  if (M == 0) {
    empty = true;
    return FD_OK;
  }
  if (!y || !hidden || !norm_w || !w || (rope_cols > 0 && (!cos || !sin)))
    return set_error(FD_EINVAL, "null pointer argument");
  if (H > 0x7fffffffLL || N > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "too large");
  if (!aligned16(hidden) || !aligned16(norm_w) || !aligned16(w))
    return set_error(FD_EUNSUPPORTED, "operands must be 16-byte aligned");
  if (mfma && (!normed || !aligned16(normed)))
    return set_error(FD_EINVAL, "M >= 5 on the MFMA path needs a 16-byte aligned normed buffer");
  e.bias = bias;
  e.bias_dtype = bias_dtype;
  e.sb = 1;
  e.row = nullptr;
  e.row_dtype = act_dtype;
  e.srm = e.srn = 0;
  rp.cos = cos;
  rp.sin = sin;
  rp.dtype = cs_dtype;
  rp.rs = cs_row_stride;
  rp.cols = (int)rope_cols;
  rp.dim = rope_cols > 0 ? (int)head_dim : 2;
  rp.tiles = 0;
  return FD_OK;
}

}  // namespace fd
