// In-process bandwidth roofs: a 16-byte-vector copy, a read of the same layout
// and a STREAM-style triad. Every percent-of-roof figure divides by the copy
// measured with these; the read is the ceiling of a kernel that only streams
// (the decode GEMVs, whose outputs are a few KiB).
// Also the library's version and error entry points.
#include "fd_device.h"
#include "fd_host.h"

namespace fd {

constexpr int kRoofThreads = 256;
constexpr int kRoofUnroll = 4;

// Each thread moves kRoofUnroll vectors, strided by the block so every load
// instruction of a wave covers 1 KiB of contiguous memory. Nontemporal loads and
// stores: the fastest copy measured on MI355X (6.1 TB/s over 2 GiB, against
// 5.7 TB/s with ordinary ones), so the roof is not understated.
__global__ __launch_bounds__(kRoofThreads) void copy_vec_kernel(u32x4* dst, const u32x4* src,
                                                                int64_t nvec) {
  const int64_t base = (int64_t)blockIdx.x * (kRoofThreads * kRoofUnroll) + threadIdx.x;
  u32x4 v[kRoofUnroll];
#pragma unroll
  for (int i = 0; i < kRoofUnroll; ++i) {
    const int64_t e = base + i * kRoofThreads;
    if (e < nvec) v[i] = __builtin_nontemporal_load(src + e);
  }
#pragma unroll
  for (int i = 0; i < kRoofUnroll; ++i) {
    const int64_t e = base + i * kRoofThreads;
    if (e < nvec) __builtin_nontemporal_store(v[i], dst + e);
  }
}

// The copy's loads alone: each thread xors its kRoofUnroll vectors, a wave
// combines its lanes, and the flag is set where a wave's result equals `key`,
// so no load can be dropped and the stores are one per 64 KiB at most.
__global__ __launch_bounds__(kRoofThreads) void read_vec_kernel(const u32x4* src, int64_t nvec,
                                                                uint32_t key, uint32_t* hit) {
  const int64_t base = (int64_t)blockIdx.x * (kRoofThreads * kRoofUnroll) + threadIdx.x;
  u32x4 v[kRoofUnroll];
#pragma unroll
  for (int i = 0; i < kRoofUnroll; ++i) {
    const int64_t e = base + i * kRoofThreads;
    v[i] = e < nvec ? __builtin_nontemporal_load(src + e) : u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < kRoofUnroll; ++i) acc ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off);
  if ((threadIdx.x & (kWave - 1)) == 0 && acc == key) atomicOr(hit, 1u);
}

__global__ __launch_bounds__(kRoofThreads) void copy_byte_kernel(uint8_t* dst, const uint8_t* src,
                                                                 int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * kRoofThreads + threadIdx.x;
  if (e < n) dst[e] = src[e];
}

template <typename T>
__global__ __launch_bounds__(kRoofThreads) void triad_vec_kernel(T* c, const T* a, const T* b,
                                                                 float scale, int64_t nvec) {
  const int64_t e = (int64_t)blockIdx.x * kRoofThreads + threadIdx.x;
  if (e >= nvec) return;
  float fa[8], fb[8];
  load8_f32<T>(a + e * 8, fa);
  load8_f32<T>(b + e * 8, fb);
  if constexpr (sizeof(T) == 4) {
    f32x4 lo, hi;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = fa[i] + fb[i] * scale;
      hi[i] = fa[i + 4] + fb[i + 4] * scale;
    }
    reinterpret_cast<f32x4*>(c + e * 8)[0] = lo;
    reinterpret_cast<f32x4*>(c + e * 8)[1] = hi;
  } else {
    typename Vec8<T>::type o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(fa[i] + fb[i] * scale);
    store8<T>(c + e * 8, o);
  }
}

template <typename T>
__global__ __launch_bounds__(kRoofThreads) void triad_tail_kernel(T* c, const T* a, const T* b,
                                                                  float scale, int64_t start,
                                                                  int64_t n) {
  const int64_t e = start + (int64_t)blockIdx.x * kRoofThreads + threadIdx.x;
  if (e < n) c[e] = from_f32<T>(to_f32(a[e]) + to_f32(b[e]) * scale);
}

}  // namespace fd

using namespace fd;

extern "C" int fd_version(void) { return 100; }

extern "C" int fd_runtime_version(int* version) {
  if (!version) return set_error(FD_EINVAL, "null pointer argument");
  if (hipRuntimeGetVersion(version) != hipSuccess)
    return set_error(FD_ELAUNCH, "hipRuntimeGetVersion failed");
  return FD_OK;
}

extern "C" const char* fd_last_error(void) { return g_last_error; }

extern "C" int fd_copy(void* dst, const void* src, int64_t bytes, void* stream) {
  if (bytes < 0) return set_error(FD_EINVAL, "bytes must be >= 0");
  if (bytes == 0) return FD_OK;
  if (!dst || !src) return set_error(FD_EINVAL, "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (aligned16(dst) && aligned16(src) && bytes % 16 == 0) {
    const int64_t nvec = bytes / 16;
    const int64_t blocks = (nvec + kRoofThreads * kRoofUnroll - 1) / (kRoofThreads * kRoofUnroll);
    if (blocks > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "copy too large");
    hipLaunchKernelGGL(copy_vec_kernel, dim3((unsigned)blocks), dim3(kRoofThreads), 0, st,
                       (u32x4*)dst, (const u32x4*)src, nvec);
  } else {
    const int64_t blocks = (bytes + kRoofThreads - 1) / kRoofThreads;
    if (blocks > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "copy too large");
    hipLaunchKernelGGL(copy_byte_kernel, dim3((unsigned)blocks), dim3(kRoofThreads), 0, st,
                       (uint8_t*)dst, (const uint8_t*)src, bytes);
  }
  return check_launch();
}

extern "C" int fd_read(const void* src, int64_t bytes, int key, void* hit, void* stream) {
  if (bytes < 0) return set_error(FD_EINVAL, "bytes must be >= 0");
  if (bytes == 0) return FD_OK;
  if (!src || !hit) return set_error(FD_EINVAL, "null pointer argument");
  if (!aligned16(src) || bytes % 16 != 0)
    return set_error(FD_EUNSUPPORTED, "the read roof needs a 16-byte aligned source and bytes %% 16 == 0");
  if ((uintptr_t)hit % 4 != 0) return set_error(FD_EINVAL, "hit must be 4-byte aligned");
  const int64_t nvec = bytes / 16;
  const int64_t blocks = (nvec + kRoofThreads * kRoofUnroll - 1) / (kRoofThreads * kRoofUnroll);
  if (blocks > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "read too large");
  hipLaunchKernelGGL(read_vec_kernel, dim3((unsigned)blocks), dim3(kRoofThreads), 0,
                     static_cast<hipStream_t>(stream), (const u32x4*)src, nvec, (uint32_t)key,
                     static_cast<uint32_t*>(hit));
  return check_launch();
}

extern "C" int fd_triad(void* c, const void* a, const void* b, float scale, int64_t n, int dtype,
                        void* stream) {
  if (!check_any_dtype(dtype, "dtype")) return FD_EINVAL;
  if (n < 0) return set_error(FD_EINVAL, "n must be >= 0");
  if (n == 0) return FD_OK;
  if (!a || !b || !c) return set_error(FD_EINVAL, "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = aligned16(a) && aligned16(b) && aligned16(c);
  const int64_t nvec = vec ? n / 8 : 0;
  const int64_t start = nvec * 8;
  if (nvec > 0) {
    const int64_t blocks = (nvec + kRoofThreads - 1) / kRoofThreads;
    if (blocks > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "triad too large");
#define FD_TRIAD(T)                                                                            \
  hipLaunchKernelGGL(triad_vec_kernel<T>, dim3((unsigned)blocks), dim3(kRoofThreads), 0, st, \
                     (T*)c, (const T*)a, (const T*)b, scale, nvec)
    if (dtype == FD_F32) FD_TRIAD(float);
    else if (dtype == FD_BF16) FD_TRIAD(bf16);
    else FD_TRIAD(f16);
#undef FD_TRIAD
  }
  if (start < n) {
    const int64_t blocks = (n - start + kRoofThreads - 1) / kRoofThreads;
    if (blocks > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "triad too large");
#define FD_TRIAD_TAIL(T)                                                                        \
  hipLaunchKernelGGL(triad_tail_kernel<T>, dim3((unsigned)blocks), dim3(kRoofThreads), 0, st, \
                     (T*)c, (const T*)a, (const T*)b, scale, start, n)
    if (dtype == FD_F32) FD_TRIAD_TAIL(float);
    else if (dtype == FD_BF16) FD_TRIAD_TAIL(bf16);
    else FD_TRIAD_TAIL(f16);
#undef FD_TRIAD_TAIL
  }
  return check_launch();
}
