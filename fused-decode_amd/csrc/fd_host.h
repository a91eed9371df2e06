// Host-side argument checking and error reporting shared by the C ABI entry
// points. Every check runs before any HIP call, so a rejected call launches
// nothing and can be tested without a GPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <cmath>

#include "fused_decode.h"

namespace fd {

inline thread_local char g_last_error[512] = "";

inline int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

inline bool check_act_dtype(int dt) {
  if (dt == FD_F16 || dt == FD_BF16) return true;
  set_error(FD_EINVAL, "act_dtype must be FD_F16 or FD_BF16, got %d", dt);
  return false;
}

inline bool check_any_dtype(int dt, const char* what) {
  if (dt == FD_F16 || dt == FD_BF16 || dt == FD_F32) return true;
  set_error(FD_EINVAL, "%s must be FD_F16, FD_BF16 or FD_F32, got %d", what, dt);
  return false;
}

inline bool check_rows(const fd_rows& l, const char* what) {
  if (l.a < 0 || l.b < 0 || l.c < 0 || l.n < 0) {
    set_error(FD_EINVAL, "%s layout has a negative size", what);
    return false;
  }
  if (l.sa < 0 || l.sb < 0 || l.sc < 0 || l.col < 0) {
    set_error(FD_EINVAL, "%s layout has a negative stride", what);
    return false;
  }
  return true;
}

inline bool same_grid(const fd_rows& x, const fd_rows& o, const char* what) {
  if (x.a != o.a || x.b != o.b || x.c != o.c || x.n != o.n) {
    set_error(FD_EINVAL, "%s cannot be indexed with the same row grid as the input", what);
    return false;
  }
  return true;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// True when the byte ranges [a, a + na) and [b, b + nb) share a byte.
inline bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return na > 0 && nb > 0 && pa < pb + (uintptr_t)nb && pb < pa + (uintptr_t)na;
}

// The MLP entry points write y and mid while hidden is still to be read (the
// down projection adds hidden as its residual, and from M = 5 y first holds the
// normalised rows): none of the three may share memory.
inline int check_mlp_buffers(const void* y, const void* mid, const void* hidden, int64_t M,
                             int64_t H, int64_t I, int elem_bytes) {
  const int64_t nh = M * H * elem_bytes, ni = M * I * elem_bytes;
  if (overlaps(y, nh, hidden, nh)) return set_error(FD_EINVAL, "y must not overlap hidden");
  if (overlaps(mid, ni, hidden, nh) || overlaps(mid, ni, y, nh))
    return set_error(FD_EINVAL, "mid must not overlap y or hidden");
  return FD_OK;
}

// True when every row of `l` is a run of n contiguous elements whose start is
// 16-byte aligned and n is a multiple of 8 (so 16-byte vectors tile the row).
inline bool rows_vectorizable(const void* p, const fd_rows& l, int elem_bytes) {
  const int64_t v = 16 / elem_bytes;
  if (!aligned16(p) || l.n % v != 0) return false;
  if (l.n > 1 && l.col != 1) return false;
  if (l.a > 1 && l.sa % v != 0) return false;
  if (l.b > 1 && l.sb % v != 0) return false;
  if (l.c > 1 && l.sc % v != 0) return false;
  return true;
}

// Row sums of squares handed between launches (a producer GEMV's per-tile sums
// of its squared outputs, read by the next RMSNorm): the checks of a *_sumsq
// entry point's `ss_in` (ceil(H/16) tiles of the norm input's width H) and
// `ss_out`. `mfma`: whether this call runs the MFMA kernels that read or write
// them.
inline int check_sumsq(bool mfma, const float* ss_in, int64_t ss_tiles, int64_t H, const float* ss_out) {
  if (!mfma)
    return set_error(FD_EUNSUPPORTED, "row sums of squares are for the MFMA kernels (kind=dot, M >= 5)");
  if (ss_in) {
    if (ss_tiles != (H + 15) / 16)
      return set_error(FD_EINVAL, "ss_tiles must be ceil(H / 16) = %lld, got %lld", (long long)((H + 15) / 16),
                       (long long)ss_tiles);
    if (!aligned16(ss_in)) return set_error(FD_EUNSUPPORTED, "ss_in must be 16-byte aligned");
  }
  if (ss_out && !aligned16(ss_out)) return set_error(FD_EUNSUPPORTED, "ss_out must be 16-byte aligned");
  return FD_OK;
}

inline int check_launch() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FD_ELAUNCH, "HIP launch failed: %s", hipGetErrorString(e));
  return FD_OK;
}

}  // namespace fd
