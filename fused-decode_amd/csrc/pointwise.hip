// Streaming elementwise kernels for gfx950: SwiGLU and rotate-half RoPE.
//
// Both run on the row grid of fd_rows (up to three leading dims with arbitrary
// strides, including 0 for broadcast operands). The vector kernels move one
// 16-byte vector per operand per thread, with nontemporal loads and stores for
// the activations (each byte is touched once); the generic kernels take any
// column stride and any row length.
#include "fd_device.h"
#include "fd_host.h"

namespace fd {

constexpr int kPwThreads = 256;

// ---------------------------------------------------------------------------
// SwiGLU: y = round(silu(g) * u), float32 math (reference.py:33-35, stable sigmoid
// as kernels.py:448-451).

template <typename T>
__global__ __launch_bounds__(kPwThreads) void swiglu_vec_kernel(T* y, const T* g, const T* u,
                                                                RowGrid grid, FastDiv vpr,
                                                                RowStrides sg, RowStrides su,
                                                                RowStrides sy, uint32_t total) {
  const uint32_t v = blockIdx.x * kPwThreads + threadIdx.x;
  if (v >= total) return;
  uint32_t cv;
  const uint32_t row = vpr.divmod(v, cv);
  const uint32_t k = cv * 8;
  const RowPos p = row_pos(grid, row);
  typename Vec8<T>::type a = load8_nt<T>(g + row_off(sg, p) + k);
  typename Vec8<T>::type b = load8_nt<T>(u + row_off(su, p) + k);
  typename Vec8<T>::type o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(silu_stable(to_f32(a[i])) * to_f32(b[i]));
  store8_nt<T>(y + row_off(sy, p) + k, o);
}

template <typename T>
__global__ __launch_bounds__(kPwThreads) void swiglu_gen_kernel(T* y, const T* g, const T* u,
                                                                RowGrid grid, FastDiv n,
                                                                RowStrides sg, RowStrides su,
                                                                RowStrides sy, uint32_t total) {
  const uint32_t e = blockIdx.x * kPwThreads + threadIdx.x;
  if (e >= total) return;
  uint32_t k;
  const uint32_t row = n.divmod(e, k);
  const RowPos p = row_pos(grid, row);
  const float a = to_f32(g[row_off(sg, p) + (int64_t)k * sg.col]);
  const float b = to_f32(u[row_off(su, p) + (int64_t)k * su.col]);
  y[row_off(sy, p) + (int64_t)k * sy.col] = from_f32<T>(silu_stable(a) * b);
}

// ---------------------------------------------------------------------------
// RoPE, rotate-half pairing (reference.py:38-47):
//   y[j]     = x[j] * c[j]     - x[j+h] * s[j]
//   y[j + h] = x[j+h] * c[j+h] + x[j] * s[j+h]

// HPT rows per thread: when cos/sin do not vary along the innermost row dim
// (stride 0 there, e.g. one table row shared by all heads of a token), a thread
// handles HPT consecutive rows of that dim and loads its cos/sin vectors once.
template <typename T, typename C, int HPT>
__global__ __launch_bounds__(kPwThreads) void rope_vec_kernel(T* y, const T* x, const C* cs,
                                                              const C* sn, RowGrid grid,
                                                              FastDiv vpr, RowStrides sx,
                                                              RowStrides sc, RowStrides ss,
                                                              RowStrides sy, uint32_t h,
                                                              uint32_t total) {
  const uint32_t v = blockIdx.x * kPwThreads + threadIdx.x;
  if (v >= total) return;
  uint32_t jv;
  const uint32_t grp = vpr.divmod(v, jv);
  const uint32_t j = jv * 8;
  const RowPos p = row_pos(grid, grp * HPT);
  const C* cr = cs + row_off(sc, p);
  const C* sr = sn + row_off(ss, p);
  float c1[8], c2[8], s1[8], s2[8];
  load8_f32<C>(cr + j, c1);
  load8_f32<C>(cr + j + h, c2);
  load8_f32<C>(sr + j, s1);
  load8_f32<C>(sr + j + h, s2);
  const T* xr = x + row_off(sx, p);
  T* yr = y + row_off(sy, p);
  typename Vec8<T>::type x1[HPT], x2[HPT];
#pragma unroll
  for (int t = 0; t < HPT; ++t) {
    x1[t] = load8_nt<T>(xr + t * sx.sc + j);
    x2[t] = load8_nt<T>(xr + t * sx.sc + j + h);
  }
#pragma unroll
  for (int t = 0; t < HPT; ++t) {
    typename Vec8<T>::type o1, o2;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float a = to_f32(x1[t][i]), b = to_f32(x2[t][i]);
      o1[i] = from_f32<T>(a * c1[i] - b * s1[i]);
      o2[i] = from_f32<T>(b * c2[i] + a * s2[i]);
    }
    store8_nt<T>(yr + t * sy.sc + j, o1);
    store8_nt<T>(yr + t * sy.sc + j + h, o2);
  }
}

template <typename T>
__global__ __launch_bounds__(kPwThreads) void rope_gen_kernel(T* y, const T* x, const void* cs,
                                                              const void* sn, int cs_dtype,
                                                              RowGrid grid, FastDiv hd,
                                                              RowStrides sx, RowStrides sc,
                                                              RowStrides ss, RowStrides sy,
                                                              uint32_t total) {
  const uint32_t e = blockIdx.x * kPwThreads + threadIdx.x;
  if (e >= total) return;
  uint32_t j;
  const uint32_t row = hd.divmod(e, j);
  const int64_t h = hd.d;
  const RowPos p = row_pos(grid, row);
  const T* xr = x + row_off(sx, p);
  const int64_t cb = row_off(sc, p), sb = row_off(ss, p);
  const float a = to_f32(xr[j * sx.col]);
  const float b = to_f32(xr[(j + h) * sx.col]);
  const float c1 = load_any(cs, cs_dtype, cb + j * sc.col);
  const float c2 = load_any(cs, cs_dtype, cb + (j + h) * sc.col);
  const float s1 = load_any(sn, cs_dtype, sb + j * ss.col);
  const float s2 = load_any(sn, cs_dtype, sb + (j + h) * ss.col);
  T* yr = y + row_off(sy, p);
  yr[j * sy.col] = from_f32<T>(a * c1 - b * s1);
  yr[(j + h) * sy.col] = from_f32<T>(b * c2 + a * s2);
}

namespace {

// Work items (vectors, elements or pairs) of one launch are counted in 32 bits.
constexpr int64_t kMaxPwWork = 0xffffffffLL - kPwThreads;

inline unsigned blocks_for(int64_t work) {
  return (unsigned)((work + kPwThreads - 1) / kPwThreads);
}

// Row layout with the last dim halved: the vector rope kernel addresses pairs
// (j, j+h), so alignment is needed at both j and h.
inline bool rope_rows_vec(const void* p, const fd_rows& l, int elem) {
  fd_rows half = l;
  half.n = l.n / 2;
  return rows_vectorizable(p, half, elem);
}

}  // namespace
}  // namespace fd

using namespace fd;

extern "C" int fd_swiglu(void* y, const void* gate, const void* up, const fd_rows* lg,
                         const fd_rows* lu, const fd_rows* ly, int act_dtype, void* stream) {
  if (!check_act_dtype(act_dtype)) return FD_EINVAL;
  if (!y || !gate || !up || !lg || !lu || !ly) return set_error(FD_EINVAL, "null pointer argument");
  if (!check_rows(*lg, "gate") || !check_rows(*lu, "up") || !check_rows(*ly, "out") ||
      !same_grid(*lg, *lu, "up") || !same_grid(*lg, *ly, "out"))
    return FD_EINVAL;
  const int64_t rows = lg->a * lg->b * lg->c;
  const int64_t total = rows * lg->n;
  if (total == 0) return FD_OK;
  if (total > kMaxPwWork) return set_error(FD_EUNSUPPORTED, "swiglu tensor too large (>= 2^32 elements)");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const RowGrid grid = row_grid(*lg);
  const bool vec = rows_vectorizable(gate, *lg, 2) && rows_vectorizable(up, *lu, 2) &&
                   rows_vectorizable(y, *ly, 2);
  if (vec) {
    const uint32_t tv = (uint32_t)(total / 8);
    const FastDiv vpr((uint32_t)(lg->n / 8));
#define FD_SWIGLU_VEC(T)                                                                       \
  hipLaunchKernelGGL(swiglu_vec_kernel<T>, dim3(blocks_for(tv)), dim3(kPwThreads), 0, st,      \
                     (T*)y, (const T*)gate, (const T*)up, grid, vpr, row_strides(*lg),         \
                     row_strides(*lu), row_strides(*ly), tv)
    if (act_dtype == FD_F16) FD_SWIGLU_VEC(f16); else FD_SWIGLU_VEC(bf16);
#undef FD_SWIGLU_VEC
  } else {
    const FastDiv nd((uint32_t)lg->n);
#define FD_SWIGLU_GEN(T)                                                                       \
  hipLaunchKernelGGL(swiglu_gen_kernel<T>, dim3(blocks_for(total)), dim3(kPwThreads), 0, st,   \
                     (T*)y, (const T*)gate, (const T*)up, grid, nd, row_strides(*lg),          \
                     row_strides(*lu), row_strides(*ly), (uint32_t)total)
    if (act_dtype == FD_F16) FD_SWIGLU_GEN(f16); else FD_SWIGLU_GEN(bf16);
#undef FD_SWIGLU_GEN
  }
  return check_launch();
}

extern "C" int fd_rope(void* y, const void* x, const void* cos, const void* sin, int cs_dtype,
                       const fd_rows* lx, const fd_rows* lc, const fd_rows* ls,
                       const fd_rows* ly, int act_dtype, void* stream) {
  if (!check_act_dtype(act_dtype) || !check_any_dtype(cs_dtype, "cs_dtype")) return FD_EINVAL;
  if (!y || !x || !cos || !sin || !lx || !lc || !ls || !ly)
    return set_error(FD_EINVAL, "null pointer argument");
  if (!check_rows(*lx, "x") || !check_rows(*lc, "cos") || !check_rows(*ls, "sin") ||
      !check_rows(*ly, "out") || !same_grid(*lx, *lc, "cos") || !same_grid(*lx, *ls, "sin") ||
      !same_grid(*lx, *ly, "out"))
    return FD_EINVAL;
  if (lx->n % 2 != 0) return set_error(FD_EINVAL, "rope last dimension must be even");
  const int64_t rows = lx->a * lx->b * lx->c;
  const int64_t h = lx->n / 2;
  const int64_t total = rows * h;
  if (total == 0) return FD_OK;
  if (total > kMaxPwWork) return set_error(FD_EUNSUPPORTED, "rope tensor too large (>= 2^32 pairs)");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const RowGrid grid = row_grid(*lx);
  const int cse = cs_dtype == FD_F32 ? 4 : 2;
  const bool vec = rope_rows_vec(x, *lx, 2) && rope_rows_vec(y, *ly, 2) &&
                   rope_rows_vec(cos, *lc, cse) && rope_rows_vec(sin, *ls, cse);
  if (vec) {
    // rows sharing cos/sin along the innermost row dim are handled 4 per thread
    const int hpt = (lc->sc == 0 && ls->sc == 0 && lx->c % 4 == 0) ? 4 : 1;
    const uint32_t tv = (uint32_t)(total / 8 / hpt);
    const FastDiv vpr((uint32_t)(h / 8));
#define FD_ROPE_VEC(T, C)                                                                       \
  do {                                                                                          \
  if (hpt == 4)                                                                                 \
    hipLaunchKernelGGL((rope_vec_kernel<T, C, 4>), dim3(blocks_for(tv)), dim3(kPwThreads), 0,   \
                       st, (T*)y, (const T*)x, (const C*)cos, (const C*)sin, grid, vpr,         \
                       row_strides(*lx), row_strides(*lc), row_strides(*ls), row_strides(*ly),  \
                       (uint32_t)h, tv);                                                        \
  else                                                                                          \
    hipLaunchKernelGGL((rope_vec_kernel<T, C, 1>), dim3(blocks_for(tv)), dim3(kPwThreads), 0,   \
                       st, (T*)y, (const T*)x, (const C*)cos, (const C*)sin, grid, vpr,         \
                       row_strides(*lx), row_strides(*lc), row_strides(*ls), row_strides(*ly),  \
                       (uint32_t)h, tv);                                                        \
  } while (0)
    if (act_dtype == FD_F16) {
      if (cs_dtype == FD_F32) FD_ROPE_VEC(f16, float);
      else if (cs_dtype == FD_BF16) FD_ROPE_VEC(f16, bf16);
      else FD_ROPE_VEC(f16, f16);
    } else {
      if (cs_dtype == FD_F32) FD_ROPE_VEC(bf16, float);
      else if (cs_dtype == FD_BF16) FD_ROPE_VEC(bf16, bf16);
      else FD_ROPE_VEC(bf16, f16);
    }
#undef FD_ROPE_VEC
  } else {
    const FastDiv hd((uint32_t)h);
#define FD_ROPE_GEN(T)                                                                         \
  hipLaunchKernelGGL(rope_gen_kernel<T>, dim3(blocks_for(total)), dim3(kPwThreads), 0, st,     \
                     (T*)y, (const T*)x, cos, sin, cs_dtype, grid, hd, row_strides(*lx),       \
                     row_strides(*lc), row_strides(*ls), row_strides(*ly), (uint32_t)total)
    if (act_dtype == FD_F16) FD_ROPE_GEN(f16); else FD_ROPE_GEN(bf16);
#undef FD_ROPE_GEN
  }
  return check_launch();
}
