// Shared pieces of the GEMV-family kernels (gemv.hip, fp8.hip): tile constants,
// the GEMV epilogue, the RMSNorm prologue of the fused kernels, and the host-side
// launch-shape helpers.
#pragma once

#include "fd_device.h"
#include "fd_host.h"

namespace fd {

constexpr int kMaxWaves = 8;      // waves per workgroup (512 threads)
constexpr int kChunk = 512;       // K elements one wave covers per SIMT step
constexpr int kUnit = 128;        // K elements of one MFMA unit (4 steps of 32)

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
  const int nt = blockDim.x, nwv = nt / kWave;
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
// (this thread's KIT 8-element slices of each hidden row and of the norm
// weight) before the caller issues its first weight loads, so the norm's loads
// are not queued behind them; norm_store reduces, rounds and stages in LDS
// from registers. Usable when H <= KIT * blockDim.x * 8 (norm_in_regs); the
// same summation order and rounding as stage_normed.
template <typename T, int MMAX, int KIT>
struct NormRegs {
  typename Vec8<T>::type h[KIT][MMAX];
  float w[KIT][8];
};

template <typename T, int MMAX, int KIT>
__device__ __forceinline__ void norm_load(NormRegs<T, MMAX, KIT>& c, const T* hidden,
                                          const void* nwp, int nw_dtype, int M, int H) {
#pragma unroll
  for (int it = 0; it < KIT; ++it) {
    const int k = (threadIdx.x + it * blockDim.x) * 8;
#pragma unroll
    for (int m = 0; m < MMAX; ++m)
      c.h[it][m] = (m < M && k < H) ? load8<T>(hidden + (int64_t)m * H + k)
                                    : typename Vec8<T>::type{};
    if (k < H) {
      load8_norm_w(nwp, nw_dtype, k, c.w[it]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) c.w[it][i] = 0.f;
    }
  }
}

template <typename T, int MMAX, int KIT>
__device__ __forceinline__ void norm_store(const NormRegs<T, MMAX, KIT>& c, T* xs,
                                           float* scratch, int M, int H, float eps) {
  const int XS = xs_stride(H);
  typedef typename Vec8<T>::type V8;
  constexpr int MP = pow2_ceil(MMAX);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nwv = blockDim.x / kWave;
  float ss[MP];
#pragma unroll
  for (int m = 0; m < MP; ++m) ss[m] = 0.f;
#pragma unroll
  for (int it = 0; it < KIT; ++it) {
#pragma unroll
    for (int m = 0; m < MMAX; ++m) {
#pragma unroll
      for (int i = 0; i < 8; ++i) ss[m] += to_f32(c.h[it][m][i]) * to_f32(c.h[it][m][i]);
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
    const int k = (tid + it * (int)blockDim.x) * 8;
    if (k < H) {
#pragma unroll
      for (int m = 0; m < MMAX; ++m) {
        if (m < M) {
          const float s = inv[m];
          V8 o;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(to_f32(c.h[it][m][i]) * s * c.w[it][i]);
          store8<T>(xs + (int64_t)m * XS + k, o);
        }
      }
    }
  }
  __syncthreads();
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

constexpr bool kNtWeights = true;           // nontemporal weight loads (measured +10-20%)
constexpr size_t kMaxLds = 160 * 1024;       // LDS per CU on gfx950

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

// Compute units of the current device (cached per device).
inline int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// Dynamic LDS of a fused kernel: the staged activations and the reduction scratch.
inline size_t fused_lds(int M, int H, size_t elem, int V) {
  return (size_t)M * xs_stride(H) * elem +
         sizeof(float) * (size_t)(V * kMaxWaves > kNormScratch ? V * kMaxWaves : kNormScratch);
}

// Workgroups of the fused kernel: each stages the normalised activations in LDS
// once and then loops over weight tiles, so the grid is what can be resident at
// once, at most `per_cu` per CU and fewer when the LDS stage is large; more would
// restage x for nothing (measured at H=4096: two 8-wave workgroups per CU).
inline int fused_grid(int tiles, size_t lds, int per_cu) {
  const int fit = (int)(kMaxLds / (lds ? lds : 1));
  const int cap = device_cus() * (fit < 1 ? 1 : fit < per_cu ? fit : per_cu);
  const int per = (tiles + cap - 1) / cap;
  return (tiles + per - 1) / per;
}

}  // namespace fd
