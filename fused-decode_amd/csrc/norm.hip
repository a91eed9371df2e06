// RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Semantics (reference src/fused_decode/reference.py:14-30):
//   rms:     y = round(x * rsqrt(mean(x^2) + eps) * w)
//   add_rms: s = x + r (float32); ro = round(s); y = round(s * rsqrt(mean(s^2) + eps) * w)
// The norm always sees the float32 sum, never the rounded residual.
//
// Three kernels:
//   rms_wave_kernel - unit column stride, n % 8 == 0, 16-byte aligned rows,
//                     n <= 8192: one wave per row, the row in registers.
//   rms_vec_kernel  - the same layouts for 8192 < n <= 16384: one 256-thread
//                     workgroup per row. Both make one HBM pass: every byte is read
//                     once and written once.
//   rms_gen_kernel  - any strides and any n: two passes over the row (the second
//                     pass re-reads through L2).
// Reduction: wave64 shuffles, then one LDS exchange across the workgroup's waves.
#include "fd_device.h"
#include "fd_host.h"
#include "fd_internal.h"

namespace fd {

template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  constexpr int NWAVE = NT / kWave;
  if (NWAVE == 1) return v;
  __syncthreads();  // `red` may still be read from a previous call
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NWAVE; ++i) s += red[i];
  return s;
}

// T: activation type; W: weight type; VPT: 8-element vectors per thread.
template <typename T, typename W, int NT, int VPT, bool ADD>
__global__ __launch_bounds__(NT) void rms_vec_kernel(T* y, T* ro, const T* x, const T* r,
                                                     const W* __restrict__ w, RowGrid grid,
                                                     RowStrides lx, RowStrides lr,
                                                     RowStrides ly, RowStrides lro, int n,
                                                     float eps) {
  __shared__ float red[NT / kWave];
  const RowPos p = row_pos(grid, blockIdx.x);
  const T* xr = x + row_off(lx, p);
  const T* rr = ADD ? r + row_off(lr, p) : nullptr;
  float v[VPT][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int k = (j * NT + threadIdx.x) * 8;
    if (k < n) {
      typename Vec8<T>::type a = load8<T>(xr + k);
      if (ADD) {
        typename Vec8<T>::type b = load8<T>(rr + k);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = to_f32(a[i]) + to_f32(b[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = to_f32(a[i]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[j][i] * v[j][i];
    }
  }
  ss = block_sum<NT>(ss, red);
  const float inv = rsqrtf(ss / (float)n + eps);
  T* yr = y + row_off(ly, p);
  T* ror = ADD ? ro + row_off(lro, p) : nullptr;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int k = (j * NT + threadIdx.x) * 8;
    if (k < n) {
      float wf[8];
      load8_f32<W>(w + k, wf);
      typename Vec8<T>::type o;
      if (ADD) {
        typename Vec8<T>::type s;
#pragma unroll
        for (int i = 0; i < 8; ++i) s[i] = from_f32<T>(v[j][i]);
        store8<T>(ror + k, s);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(v[j][i] * inv * wf[i]);
      store8<T>(yr + k, o);
    }
  }
}

// One wave per row, four rows per workgroup: the reduction is wave shuffles
// only, and each lane keeps VPL vectors of its row in registers. Activations
// stream through nontemporal loads and stores (read and written exactly once).
// The norm weight (n * sizeof(W) bytes, L2-resident, shared by every row) is
// staged once per workgroup in LDS: its loads go out before the row's, and the
// output pass reads it from LDS, so it holds no registers while the row loads
// are in flight. Without the residual the kernel is held to 64 VGPRs up to n =
// 4096 (the row packed, widened again in the output pass), so eight waves per
// SIMD keep every row of an 8192 x 4096 norm resident at once.
template <typename W>
__host__ __device__ constexpr int norm_w_chunks_per_thread(int vpl) {
  return vpl * (int)sizeof(W) / 8 > 0 ? vpl * (int)sizeof(W) / 8 : 1;  // n <= vpl * 512
}

template <typename T, typename W, int VPL, bool ADD>
__global__ __launch_bounds__(256, !ADD && VPL <= 8 ? 8 : 1) void rms_wave_kernel(T* y, T* ro, const T* x, const T* r,
                                                      const W* __restrict__ w, RowGrid grid,
                                                      RowStrides lx, RowStrides lr,
                                                      RowStrides ly, RowStrides lro, int n,
                                                      uint32_t rows, float eps) {
  typedef typename Vec8<T>::type V8;
  constexpr int WPT = norm_w_chunks_per_thread<W>(VPL);
  extern __shared__ __align__(16) u32x4 wsm[];  // the norm weight, n * sizeof(W) bytes
  const int wchunks = n * (int)sizeof(W) / 16;
  const u32x4* wsrc = reinterpret_cast<const u32x4*>(w);
  u32x4 wr[WPT];
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    const int c = threadIdx.x + i * 256;
    wr[i] = wsrc[c < wchunks ? c : 0];
  }
  const uint32_t row = blockIdx.x * 4 + threadIdx.x / kWave;
  const bool live = row < rows;  // the last workgroup's waves past the rows only stage the weight
  const int lane = threadIdx.x & (kWave - 1);
  const RowPos p = row_pos(grid, live ? row : 0);
  const T* xr = x + row_off(lx, p);
  const T* rr = ADD ? r + row_off(lr, p) : nullptr;
  V8 a[VPL], b[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int k = (j * kWave + lane) * 8;
    if (live && k < n) {
      a[j] = load8_nt<T>(xr + k);
      if (ADD) b[j] = load8_nt<T>(rr + k);
    }
  }
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c < wchunks) wsm[c] = wr[i];
  }
  __syncthreads();
  if (!live) return;
  // rms: the row stays packed in registers and its packed pairs are squared
  // with v_dot2, so nothing is widened before the output pass; add_rms keeps
  // the float32 sums x + r and writes residual_out = round(sum) in the first
  // pass (it does not depend on the norm), so those stores overlap the reduction.
  float v[ADD ? VPL : 1][8];
  float ss = 0.f;
  T* ror = ADD ? ro + row_off(lro, p) : nullptr;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int k = (j * kWave + lane) * 8;
    if (k >= n) continue;
    if constexpr (ADD) {
      V8 s;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[j][i] = to_f32(a[j][i]) + to_f32(b[j][i]);
        ss += v[j][i] * v[j][i];
        s[i] = from_f32<T>(v[j][i]);
      }
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, s), reinterpret_cast<u32x4*>(ror + k));
    } else {
      const u32x4 pk = __builtin_bit_cast(u32x4, a[j]);
#pragma unroll
      for (int i = 0; i < 4; ++i) ss = sq_dot2<T>(pk[i], ss);
    }
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)n + eps);
  T* yr = y + row_off(ly, p);
  const W* wl = reinterpret_cast<const W*>(wsm);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int k = (j * kWave + lane) * 8;
    if (k < n) {
      Raw8<W> wv;
      wv.load(wl + k);
      V8 o;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = ADD ? v[ADD ? j : 0][i] : to_f32(a[j][i]);
        o[i] = from_f32<T>(x * inv * wv[i]);
      }
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), reinterpret_cast<u32x4*>(yr + k));
    }
  }
}

template <typename T, bool ADD>
__global__ __launch_bounds__(256) void rms_gen_kernel(T* y, T* ro, const T* x, const T* r,
                                                      const void* __restrict__ w, int w_dtype,
                                                      int64_t w_stride, RowGrid grid,
                                                      RowStrides lx, RowStrides lr,
                                                      RowStrides ly, RowStrides lro, int64_t n,
                                                      float eps) {
  __shared__ float red[4];
  const RowPos p = row_pos(grid, blockIdx.x);
  const T* xr = x + row_off(lx, p);
  const T* rr = ADD ? r + row_off(lr, p) : nullptr;
  float ss = 0.f;
  for (int64_t k = threadIdx.x; k < n; k += 256) {
    float s = to_f32(xr[k * lx.col]);
    if (ADD) s += to_f32(rr[k * lr.col]);
    ss += s * s;
  }
  ss = block_sum<256>(ss, red);
  const float inv = rsqrtf(ss / (float)n + eps);
  T* yr = y + row_off(ly, p);
  T* ror = ADD ? ro + row_off(lro, p) : nullptr;
  for (int64_t k = threadIdx.x; k < n; k += 256) {
    float s = to_f32(xr[k * lx.col]);
    if (ADD) {
      s += to_f32(rr[k * lr.col]);
      ror[k * lro.col] = from_f32<T>(s);
    }
    yr[k * ly.col] = from_f32<T>(s * inv * load_any(w, w_dtype, k * w_stride));
  }
}

namespace {

template <typename T, typename W, int VPT, bool ADD>
void launch_vec(void* y, void* ro, const void* x, const void* r, const void* w,
                const fd_rows& lx, const fd_rows& lr, const fd_rows& ly, const fd_rows& lro,
                int64_t rows, float eps, hipStream_t st) {
  constexpr int NT = 256;
  hipLaunchKernelGGL((rms_vec_kernel<T, W, NT, VPT, ADD>), dim3((unsigned)rows), dim3(NT), 0,
                     st, static_cast<T*>(y), static_cast<T*>(ro), static_cast<const T*>(x),
                     static_cast<const T*>(r), static_cast<const W*>(w), row_grid(lx),
                     row_strides(lx), row_strides(lr), row_strides(ly), row_strides(lro),
                     (int)lx.n, eps);
}

template <typename T, typename W, int VPL, bool ADD>
void launch_wave(void* y, void* ro, const void* x, const void* r, const void* w,
                 const fd_rows& lx, const fd_rows& lr, const fd_rows& ly, const fd_rows& lro,
                 int64_t rows, float eps, hipStream_t st) {
  const size_t lds = (size_t)(lx.n * (int64_t)sizeof(W) + 15) / 16 * 16;  // the staged norm weight
  hipLaunchKernelGGL((rms_wave_kernel<T, W, VPL, ADD>), dim3((unsigned)((rows + 3) / 4)),
                     dim3(256), lds, st, static_cast<T*>(y), static_cast<T*>(ro),
                     static_cast<const T*>(x), static_cast<const T*>(r),
                     static_cast<const W*>(w), row_grid(lx), row_strides(lx), row_strides(lr),
                     row_strides(ly), row_strides(lro), (int)lx.n, (uint32_t)rows, eps);
}

template <typename T, typename W, bool ADD>
void pick_vpt(void* y, void* ro, const void* x, const void* r, const void* w,
              const fd_rows& lx, const fd_rows& lr, const fd_rows& ly, const fd_rows& lro,
              int64_t rows, float eps, hipStream_t st) {
  // Rows up to 8192 elements: one wave per row (VPL vectors per lane).
  const int64_t lanes_vecs = (lx.n + 8 * kWave - 1) / (8 * kWave);
  if (lanes_vecs <= 2) {
    launch_wave<T, W, 2, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
    return;
  }
  if (lanes_vecs <= 4) {
    launch_wave<T, W, 4, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
    return;
  }
  if (lanes_vecs <= 8) {
    launch_wave<T, W, 8, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
    return;
  }
  if (lanes_vecs <= 16) {
    launch_wave<T, W, 16, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
    return;
  }
  const int64_t vecs = (lx.n + 8 * 256 - 1) / (8 * 256);
  if (vecs <= 1)
    launch_vec<T, W, 1, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
  else if (vecs <= 2)
    launch_vec<T, W, 2, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
  else if (vecs <= 4)
    launch_vec<T, W, 4, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
  else
    launch_vec<T, W, 8, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
}

template <typename T, bool ADD>
void dispatch_w(int w_dtype, void* y, void* ro, const void* x, const void* r, const void* w,
                const fd_rows& lx, const fd_rows& lr, const fd_rows& ly, const fd_rows& lro,
                int64_t rows, float eps, hipStream_t st) {
  if (w_dtype == FD_F32)
    pick_vpt<T, float, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
  else if (w_dtype == FD_BF16)
    pick_vpt<T, bf16, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
  else
    pick_vpt<T, f16, ADD>(y, ro, x, r, w, lx, lr, ly, lro, rows, eps, st);
}

constexpr int64_t kVecMaxN = 256 * 8 * 8;

bool vec_ok(const void* p, const fd_rows& l, int elem) {
  return rows_vectorizable(p, l, elem) && l.n <= kVecMaxN;
}

int rms_common(bool add, void* y, void* ro, const void* x, const void* r, const void* w,
               int w_dtype, int64_t w_stride, const fd_rows* lx, const fd_rows* lr,
               const fd_rows* ly, const fd_rows* lro, float eps, int act_dtype, void* stream) {
  if (!check_act_dtype(act_dtype) || !check_any_dtype(w_dtype, "w_dtype")) return FD_EINVAL;
  if (!y || !x || !w || !lx || !ly) return set_error(FD_EINVAL, "null pointer argument");
  if (add && (!ro || !r || !lr || !lro)) return set_error(FD_EINVAL, "null residual argument");
  if (!check_rows(*lx, "x") || !check_rows(*ly, "out") || !same_grid(*lx, *ly, "out"))
    return FD_EINVAL;
  if (add && (!check_rows(*lr, "residual") || !check_rows(*lro, "residual_out") ||
              !same_grid(*lx, *lr, "residual") || !same_grid(*lx, *lro, "residual_out")))
    return FD_EINVAL;
  if (!(eps >= 0.f) || eps == INFINITY) return set_error(FD_EINVAL, "eps must be a finite value >= 0");
  const int64_t rows = lx->a * lx->b * lx->c;
  if (rows == 0 || lx->n == 0) return FD_OK;
  if (rows > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "too many rows (>= 2^31)");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const fd_rows& LR = add ? *lr : *lx;
  const fd_rows& LRO = add ? *lro : *ly;
  const int wsz = w_dtype == FD_F32 ? 4 : 2;
  bool vec = vec_ok(x, *lx, 2) && vec_ok(y, *ly, 2) && w_stride == 1 &&
             (reinterpret_cast<uintptr_t>(w) % 16) == 0;
  (void)wsz;
  if (add) vec = vec && vec_ok(r, *lr, 2) && vec_ok(ro, *lro, 2);
  if (vec) {
    if (act_dtype == FD_F16) {
      if (add)
        dispatch_w<f16, true>(w_dtype, y, ro, x, r, w, *lx, LR, *ly, LRO, rows, eps, st);
      else
        dispatch_w<f16, false>(w_dtype, y, ro, x, r, w, *lx, LR, *ly, LRO, rows, eps, st);
    } else {
      if (add)
        dispatch_w<bf16, true>(w_dtype, y, ro, x, r, w, *lx, LR, *ly, LRO, rows, eps, st);
      else
        dispatch_w<bf16, false>(w_dtype, y, ro, x, r, w, *lx, LR, *ly, LRO, rows, eps, st);
    }
  } else {
#define FD_RMS_GEN(T, A)                                                                     \
  hipLaunchKernelGGL((rms_gen_kernel<T, A>), dim3((unsigned)rows), dim3(256), 0, st,         \
                     static_cast<T*>(y), static_cast<T*>(ro), static_cast<const T*>(x),      \
                     static_cast<const T*>(r), w, w_dtype, w_stride, row_grid(*lx),          \
                     row_strides(*lx), row_strides(LR), row_strides(*ly), row_strides(LRO),   \
                     lx->n, eps)
    if (act_dtype == FD_F16) {
      if (add) FD_RMS_GEN(f16, true); else FD_RMS_GEN(f16, false);
    } else {
      if (add) FD_RMS_GEN(bf16, true); else FD_RMS_GEN(bf16, false);
    }
#undef FD_RMS_GEN
  }
  return check_launch();
}

}  // namespace

int rms_rows(void* y, const void* x, const void* w, int w_dtype, int64_t rows, int64_t n,
             float eps, int act_dtype, hipStream_t st) {
  fd_rows l;
  l.a = 1;
  l.b = 1;
  l.c = rows;
  l.sa = 0;
  l.sb = 0;
  l.sc = n;
  l.col = 1;
  l.n = n;
  return rms_common(false, y, nullptr, x, nullptr, w, w_dtype, 1, &l, nullptr, &l, nullptr, eps,
                    act_dtype, st);
}

}  // namespace fd

extern "C" int fd_rms_norm(void* y, const void* x, const void* w, int w_dtype, int64_t w_stride,
                           const fd_rows* lx, const fd_rows* ly, float eps, int act_dtype,
                           void* stream) {
  return fd::rms_common(false, y, nullptr, x, nullptr, w, w_dtype, w_stride, lx, nullptr, ly,
                        nullptr, eps, act_dtype, stream);
}

extern "C" int fd_add_rms_norm(void* y, void* residual_out, const void* x, const void* residual,
                               const void* w, int w_dtype, int64_t w_stride, const fd_rows* lx,
                               const fd_rows* lr, const fd_rows* ly, const fd_rows* lro,
                               float eps, int act_dtype, void* stream) {
  return fd::rms_common(true, y, residual_out, x, residual, w, w_dtype, w_stride, lx, lr, ly,
                        lro, eps, act_dtype, stream);
}
