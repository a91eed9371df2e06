// Device-side helpers shared by the gfx950 kernels: element types, 16-byte
// vector loads/stores, float conversions, the row-layout index, and wave64
// reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fd_fastdiv.h"
#include "fused_decode.h"

namespace fd {

typedef _Float16 f16;
typedef __bf16 bf16;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Threads per workgroup. Every launch in this library uses whole workgroups,
// so this is the dispatch's workgroup size, read at a fixed offset with a
// scalar load. blockDim.x also selects the partial-workgroup remainder; the
// compiler folds that select into a 2-byte vector load at a variable offset,
// re-issues it at each use, and its vmcnt wait then also waits for every
// weight load already in flight.
__device__ __forceinline__ int block_threads() { return __builtin_amdgcn_workgroup_size_x(); }

// 8 activation elements = one 16-byte vector.
template <typename T> struct Vec8;
template <> struct Vec8<f16> { typedef f16x8 type; };
template <> struct Vec8<bf16> { typedef bf16x8 type; };

__device__ __forceinline__ float to_f32(f16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(float v) { return v; }

// Round-to-nearest-even float32 -> storage type (the same rounding as torch's .to()).
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return (f16)v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }

// Round-trip through the storage type: the value a stored-then-reloaded tensor holds.
template <typename T> __device__ __forceinline__ float round_as(float v) {
  return to_f32(from_f32<T>(v));
}

// 16-byte load of 8 activations (pointer must be 16-byte aligned).
template <typename T>
__device__ __forceinline__ typename Vec8<T>::type load8(const T* p) {
  return *reinterpret_cast<const typename Vec8<T>::type*>(p);
}
// 16-byte load that bypasses cache retention (nontemporal): for weight streams
// read exactly once, so they do not evict operands that are reused.
template <typename T>
__device__ __forceinline__ typename Vec8<T>::type load8_nt(const T* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return __builtin_bit_cast(typename Vec8<T>::type, v);
}
// Weight load: nontemporal when NT.
template <bool NT, typename T>
__device__ __forceinline__ typename Vec8<T>::type load8w(const T* p) {
  if constexpr (NT)
    return load8_nt<T>(p);
  else
    return load8<T>(p);
}
// 16-byte store that does not retain the line (for outputs written once).
template <typename T>
__device__ __forceinline__ void store8_nt(T* p, typename Vec8<T>::type v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(p));
}
template <typename T>
__device__ __forceinline__ void store8(T* p, typename Vec8<T>::type v) {
  *reinterpret_cast<typename Vec8<T>::type*>(p) = v;
}

// 8 consecutive values of any of the three dtypes, widened to float32.
template <typename W>
__device__ __forceinline__ void load8_f32(const W* p, float (&f)[8]) {
  typename Vec8<W>::type v = load8<W>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = to_f32(v[i]);
}
template <>
__device__ __forceinline__ void load8_f32<float>(const float* p, float (&f)[8]) {
  f32x4 a = *reinterpret_cast<const f32x4*>(p);
  f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = a[i];
    f[i + 4] = b[i];
  }
}

// 8 consecutive values of any of the three dtypes kept in their storage form
// (4 VGPRs for fp16/bf16, 8 for fp32) and widened one element at a time.
template <typename W> struct Raw8 {
  typename Vec8<W>::type v;
  __device__ __forceinline__ void load(const W* p) { v = load8<W>(p); }
  __device__ __forceinline__ float operator[](int i) const { return to_f32(v[i]); }
};
template <> struct Raw8<float> {
  f32x4 lo, hi;
  __device__ __forceinline__ void load(const float* p) {
    lo = *reinterpret_cast<const f32x4*>(p);
    hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ float operator[](int i) const { return i < 4 ? lo[i] : hi[i - 4]; }
};

// Scalar load of element `i` of a buffer whose dtype is known only at run time.
__device__ __forceinline__ float load_any(const void* p, int dtype, int64_t i) {
  if (dtype == FD_F32) return static_cast<const float*>(p)[i];
  if (dtype == FD_BF16) return to_f32(static_cast<const bf16*>(p)[i]);
  return to_f32(static_cast<const f16*>(p)[i]);
}

// Row grid shared by every operand of a launch: linear row r is (a, b, c) with
// c = r % C, b = (r / C) % B, a = r / (C * B). Divisions by the launch-fixed
// C and B use FastDiv (multiply-high + shift), computed once per thread.
struct RowGrid {
  FastDiv c, b;
};
// Per-operand strides (elements) of the three row dims and of the columns.
struct RowStrides {
  int64_t sa, sb, sc, col;
};
struct RowPos {
  uint32_t a, b, c;
};

inline RowGrid row_grid(const fd_rows& l) {
  RowGrid g;
  g.c = FastDiv((uint32_t)l.c);
  g.b = FastDiv((uint32_t)l.b);
  return g;
}

inline RowStrides row_strides(const fd_rows& l) {
  RowStrides s;
  s.sa = l.sa;
  s.sb = l.sb;
  s.sc = l.sc;
  s.col = l.col;
  return s;
}

__device__ __forceinline__ RowPos row_pos(const RowGrid& g, uint32_t row) {
  RowPos p;
  const uint32_t t = g.c.divmod(row, p.c);
  p.a = g.b.divmod(t, p.b);
  return p;
}

// Offset (elements) of the first element of the row at `p`.
__device__ __forceinline__ int64_t row_off(const RowStrides& s, const RowPos& p) {
  return (int64_t)p.a * s.sa + (int64_t)p.b * s.sb + (int64_t)p.c * s.sc;
}

// Dot product of 8 activation pairs accumulated into float32 with v_dot2
// (each fp16/bf16 product is exact in float32).
__device__ __forceinline__ float dot8(f16x8 a, f16x8 b, float acc) {
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 0, 1),
                               __builtin_shufflevector(b, b, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 2, 3),
                               __builtin_shufflevector(b, b, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 4, 5),
                               __builtin_shufflevector(b, b, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 6, 7),
                               __builtin_shufflevector(b, b, 6, 7), acc, false);
  return acc;
}
__device__ __forceinline__ float dot8(bf16x8 a, bf16x8 b, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 0, 1),
                                        __builtin_shufflevector(b, b, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 2, 3),
                                        __builtin_shufflevector(b, b, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 4, 5),
                                        __builtin_shufflevector(b, b, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 6, 7),
                                        __builtin_shufflevector(b, b, 6, 7), acc, false);
  return acc;
}

// dot8(a, b, 0.f) with the first pair's product taken by the VOP3P form of
// v_dot2 and an inline-constant zero addend, so no register is zeroed first
// (the compiler otherwise zeroes one and uses v_dot2c). The same sums in the
// same order as dot8.
__device__ __forceinline__ float dot8_first(f16x8 a, f16x8 b) {
  const u32x4 ua = __builtin_bit_cast(u32x4, a), ub = __builtin_bit_cast(u32x4, b);
  float acc;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(acc) : "v"(ua[0]), "v"(ub[0]));
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 2, 3),
                               __builtin_shufflevector(b, b, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 4, 5),
                               __builtin_shufflevector(b, b, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 6, 7),
                               __builtin_shufflevector(b, b, 6, 7), acc, false);
  return acc;
}
__device__ __forceinline__ float dot8_first(bf16x8 a, bf16x8 b) {
  const u32x4 ua = __builtin_bit_cast(u32x4, a), ub = __builtin_bit_cast(u32x4, b);
  float acc;
  asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(acc) : "v"(ua[0]), "v"(ub[0]));
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 2, 3),
                                        __builtin_shufflevector(b, b, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 4, 5),
                                        __builtin_shufflevector(b, b, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 6, 7),
                                        __builtin_shufflevector(b, b, 6, 7), acc, false);
  return acc;
}

// acc + the squares of the two T values packed in `pair`, in float32.
template <typename T>
__device__ __forceinline__ float sq_dot2(uint32_t pair, float acc) {
  if constexpr (std::is_same<T, f16>::value) {
    const f16x2 v = __builtin_bit_cast(f16x2, pair);
    return __builtin_amdgcn_fdot2(v, v, acc, false);
  } else {
    const bf16x2 v = __builtin_bit_cast(bf16x2, pair);
    return __builtin_amdgcn_fdot2_f32_bf16(v, v, acc, false);
  }
}

// 16x16x32 MFMA: D[16x16] += A[16x32] * B[32x16], float32 accumulate.
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Cross-lane exchanges of the reductions below, none through LDS (a shuffle is
// a ds_bpermute round trip). The partner of lane l at lane bit b is l ^ 32
// (v_permlane32_swap), l ^ 16 (v_permlane16_swap), l ^ 15 (DPP row_mirror),
// l ^ 7 (row_half_mirror), l ^ 2 and l ^ 1 (quad_perm): each flips bit b and at
// most lower bits, so partners agree on every higher bit, and exchanges taken
// over the bits from 32 down to 1 still combine all 64 lanes.
template <int MASK> struct XlaneDpp;
template <> struct XlaneDpp<8> { static constexpr int ctrl = 0x140; };  // row_mirror
template <> struct XlaneDpp<4> { static constexpr int ctrl = 0x141; };  // row_half_mirror
template <> struct XlaneDpp<2> { static constexpr int ctrl = 0x4e; };   // quad_perm 2,3,0,1
template <> struct XlaneDpp<1> { static constexpr int ctrl = 0xb1; };   // quad_perm 1,0,3,2

template <int MASK>
__device__ __forceinline__ float xlane_dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), XlaneDpp<MASK>::ctrl, 0xf, 0xf,
                                      false));
}

// Lanes with bit MASK clear return lo + the partner's lo, lanes with it set
// hi + the partner's hi. v_permlane32_swap exchanges lanes 32-63 of its first
// operand with lanes 0-31 of its second, v_permlane16_swap the odd 16-lane
// rows of its first with the even rows of its second: afterwards a lane with
// the bit clear holds its own lo and the partner's lo, a lane with it set the
// partner's hi and its own hi.
template <int MASK>
__device__ __forceinline__ float xlane_keep_sum(float lo, float hi, int lane) {
  if constexpr (MASK >= 16) {
    const unsigned a = __builtin_bit_cast(unsigned, lo), b = __builtin_bit_cast(unsigned, hi);
    const auto r = MASK == 32 ? __builtin_amdgcn_permlane32_swap(a, b, false, false)
                              : __builtin_amdgcn_permlane16_swap(a, b, false, false);
    // Copy both results out before any cast: __builtin_bit_cast applied to
    // r[1] directly reads element 0 (this clang).
    const unsigned r0 = r[0], r1 = r[1];
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
  } else {
    const bool upper = (lane & MASK) != 0;
    return (upper ? hi : lo) + xlane_dpp<MASK>(upper ? lo : hi);
  }
}

// v + the partner's v; both partners compute the same sum.
template <int MASK>
__device__ __forceinline__ float xlane_sum(float v) {
  if constexpr (MASK >= 16) {
    return xlane_keep_sum<MASK>(v, v, 0);
  } else {
    return v + xlane_dpp<MASK>(v);
  }
}

// The value lane l ^ 32 holds.
__device__ __forceinline__ float xlane_partner32(float v, int lane) {
  const unsigned a = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane32_swap(a, a, false, false);
  const unsigned r0 = r[0], r1 = r[1];  // copied out first, as in xlane_keep_sum
  return __builtin_bit_cast(float, lane < 32 ? r1 : r0);
}

// Sum over the wave's 64 lanes, identical in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v = xlane_sum<32>(v);
  v = xlane_sum<16>(v);
  v = xlane_sum<8>(v);
  v = xlane_sum<4>(v);
  v = xlane_sum<2>(v);
  return xlane_sum<1>(v);
}

// Transposing butterfly: V (a power of two <= 64) per-lane partial sums become
// V wave-wide sums using V-1 exchanges instead of 6*V. Afterwards v[0] of lane
// `l` holds the full sum of value index butterfly_index<V>(l).
// One exchange step: COUNT live values, partner = the lane across bit MASK
// (xlane_keep_sum). The lane with the bit clear keeps the lower half of the
// values, its partner the upper half; each adds the partner's copy of the half
// it keeps.
template <int V, int COUNT, int MASK>
struct Butterfly {
  static __device__ __forceinline__ void run(float (&v)[V], int lane) {
    constexpr int HALF = COUNT / 2;
#pragma unroll
    for (int i = 0; i < HALF; ++i) v[i] = xlane_keep_sum<MASK>(v[i], v[i + HALF], lane);
    Butterfly<V, HALF, MASK / 2>::run(v, lane);
  }
};
// One value left: plain reduction over the remaining lane bits.
template <int V, int MASK>
struct Butterfly<V, 1, MASK> {
  static __device__ __forceinline__ void run(float (&v)[V], int lane) {
    v[0] = xlane_sum<MASK>(v[0]);
    Butterfly<V, 1, MASK / 2>::run(v, lane);
  }
};
template <int V, int COUNT>
struct Butterfly<V, COUNT, 0> {
  static __device__ __forceinline__ void run(float (&)[V], int) {}
};
template <int V>
struct Butterfly<V, 1, 0> {
  static __device__ __forceinline__ void run(float (&)[V], int) {}
};

template <int V>
__device__ __forceinline__ void butterfly_sum(float (&v)[V], int lane) {
  static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of two <= 64");
  Butterfly<V, V, 32>::run(v, lane);
}

// Value index whose wave-wide sum lane `lane` holds after butterfly_sum<V>.
template <int V>
__device__ __forceinline__ int butterfly_index(int lane) {
  // The first log2(V) exchange masks are 32, 16, ...: lane bit (5 - s) selects the
  // upper half at step s, contributing V >> (s + 1).
  int idx = 0;
  int count = V;
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) {
    if (count > 1) {
      if (lane & mask) idx += count >> 1;
      count >>= 1;
    }
  }
  return idx;
}

// Lanes that write a distinct value after butterfly_sum<V>: one per value index.
template <int V>
__device__ __forceinline__ bool butterfly_writer(int lane) {
  // Value index bits come from the top log2(V) lane bits; the low bits are free.
  constexpr int low = 64 / V;  // lanes sharing one value
  return (lane & (low - 1)) == 0;
}

__device__ __forceinline__ float silu_stable(float g) {
  // sigmoid(g) without overflow: exp of a non-positive argument only.
  float e = __expf(-fabsf(g));
  float sig = g >= 0.f ? 1.f / (1.f + e) : e / (1.f + e);
  return g * sig;
}

}  // namespace fd
