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

// The copy's persistent form: a fixed grid walks the vectors grid-stride, each
// thread moving kRoofUnroll of them per pass (loads, then stores). Measured
// faster than copy_vec_kernel's one-pass grid on copies of 30-120 MB (33.6 MB:
// 6.0 against 7.1 us with 8 workgroups per CU), slower at 1 GiB, so it is a
// second candidate for a kernel's same-size copy ceiling, not the roof.
__global__ __launch_bounds__(kRoofThreads) void copy_persist_kernel(u32x4* dst, const u32x4* src,
                                                                    int64_t nvec) {
  const int64_t stride = (int64_t)gridDim.x * (kRoofThreads * kRoofUnroll);
  for (int64_t base = (int64_t)blockIdx.x * (kRoofThreads * kRoofUnroll) + threadIdx.x; base < nvec;
       base += stride) {
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

// Clock probe: lane 0 of each workgroup records where it ran -- its XCD's id
// and its CU's position in it (the SE, SH and CU fields of HW_ID) in one word --
// the shader clock counter (s_memtime) and the constant-rate wall clock
// (s_memrealtime). The shader counters of different CUs are not synchronised,
// so two probes on one stream around a piece of work are compared CU by CU:
// a CU's counter advance over the wall clock's is proportional to its gfx
// clock during the work.
__global__ __launch_bounds__(64) void clock_probe_kernel(unsigned long long* out) {
  if (threadIdx.x == 0) {
    unsigned xcc, hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    const unsigned long long t = __builtin_amdgcn_s_memtime();
    const unsigned long long w = __builtin_amdgcn_s_memrealtime();
    out[3 * blockIdx.x] = ((unsigned long long)(xcc & 0xfu) << 8) | ((hw >> 8) & 0xffu);
    out[3 * blockIdx.x + 1] = t;
    out[3 * blockIdx.x + 2] = w;
  }
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

extern "C" int fd_copy_persistent(void* dst, const void* src, int64_t bytes, int workgroups, void* stream) {
  if (bytes < 0) return set_error(FD_EINVAL, "bytes must be >= 0");
  if (workgroups < 1) return set_error(FD_EINVAL, "workgroups must be >= 1");
  if (bytes == 0) return FD_OK;
  if (!dst || !src) return set_error(FD_EINVAL, "null pointer argument");
  if (!aligned16(dst) || !aligned16(src) || bytes % 16 != 0)
    return set_error(FD_EUNSUPPORTED, "the persistent copy needs 16-byte aligned pointers and bytes %% 16 == 0");
  hipLaunchKernelGGL(copy_persist_kernel, dim3((unsigned)workgroups), dim3(kRoofThreads), 0,
                     static_cast<hipStream_t>(stream), (u32x4*)dst, (const u32x4*)src, bytes / 16);
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

extern "C" int fd_clock_probe(unsigned long long* out, int workgroups, int* wall_khz, void* stream) {
  if (!out || !wall_khz) return set_error(FD_EINVAL, "null pointer argument");
  if (workgroups < 1 || workgroups > 4096) return set_error(FD_EINVAL, "workgroups must be in [1, 4096]");
  if ((uintptr_t)out % 8 != 0) return set_error(FD_EINVAL, "out must be 8-byte aligned");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(wall_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    return set_error(FD_ELAUNCH, "cannot read the wall clock rate");
  hipLaunchKernelGGL(clock_probe_kernel, dim3((unsigned)workgroups), dim3(64), 0, static_cast<hipStream_t>(stream),
                     out);
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
