// Persistent MFMA gate/up with resident activations, for 5-8 activation rows
// (the MLP's fused RMSNorm + gate/up + SwiGLU). Written for fp16/bf16 and E4M3
// weights; the library launches it for E4M3 weights (with fp16/bf16 weights it
// ties the relayout kernel).
//
// One workgroup per CU walks the tiles blockIdx.x, blockIdx.x + gridDim.x, ...
// of the gate/up weights [2I, K]: tile t is gate rows 8t..8t+7 and up rows
// I+8t..I+8t+7, the 16 rows of one v_mfma_f32_16x16x32 tile. The prologue
// moves the 8 activation rows and the norm weight into LDS by DMA, normalises
// the rows there once (round(x * inv_rms * w), inv_rms from x itself), and the
// loop then streams only weights: wave w takes K units w, w + NW, ... of every
// tile through its ring of D slots (the DMA kernel's layout and swizzle), the
// stream running on across tile boundaries, and reads its B fragments from the
// resident rows. At M = 8 the per-unit activation re-reads of the one-tile
// workgroups are half (E4M3) or a third (fp16) of the L2 requests a CU keeps
// outstanding, which the weight stream then cannot use; resident rows are read
// from L2 once per CU.
//
// Layout of the resident rows: row r holds its 16-byte chunks with chunk c at
// slot c ^ (r & 7), so the 8 lanes of a B read (8 rows, one chunk) hit distinct
// bank groups. Rows past M copy row 0 and get inv_rms 0 (zero B columns, never
// stored). K is a multiple of 512, so no unit or DMA instruction crosses it.
//
// At the end of a tile every wave leaves its partial sums in one of two LDS
// buffers (consecutive tiles alternate; they take the norm weight's place once
// the rows are normalised) and meets the others at a barrier;
// wave (tile iteration mod NW) then adds them and writes the SwiGLU outputs
// while the other waves go on with the next tile. Every LDS access in the
// prologue and the loop is inline assembly with explicit waits, and the
// barriers carry no memory fence: the compiler orders a DMA against LDS
// accesses it can see only by vmcnt(0), which would drain the weight stream.
#pragma once

#include "fd_dma.h"

namespace fd {

constexpr int kResRows = 8;    // activation rows staged (M <= 8)
constexpr int kResMaxTiles = 16;  // tiles per workgroup (E4M3 row scales staged for these)

// Dynamic LDS of a launch for K padded to whole units (kp) and nw waves: the
// resident rows; one region that holds the norm weight (room for float32)
// during the prologue and the two partial-sum buffers after it; the E4M3 row
// scales of up to kResMaxTiles tiles (one DMA instruction).
__host__ __device__ constexpr size_t res_shared_bytes(int kp, int nw) {
  return (size_t)kp * 4 > (size_t)2 * nw * kWave * 16 ? (size_t)kp * 4 : (size_t)2 * nw * kWave * 16;
}
__host__ __device__ constexpr size_t res_dyn_lds(int kp, int nw) {
  return (size_t)kResRows * kp * 2 + res_shared_bytes(kp, nw) + (size_t)kWave * 16;
}
// Static LDS: the rings.
__host__ __device__ constexpr size_t res_static_lds(int nw, int d, int wbytes) {
  return (size_t)nw * d * dma_geom(wbytes).ae * 16;
}

// Make NR ds_read results usable: one s_waitcnt lgkmcnt(0), then an empty
// statement per register that claims to rewrite it, so no use of a result is
// scheduled ahead of the wait (volatile statements keep their order).
template <int NR>
__device__ __forceinline__ void res_wait_lds(u32x4 (&v)[NR]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < NR; ++i) asm volatile("" : "+v"(v[i]));
}

__device__ __forceinline__ void res_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}

template <typename T, typename W, int NW, int D>
__global__ __launch_bounds__(NW * kWave) void gate_up_res_kernel(T* mid, const T* x, const W* w,
                                                                 const float* wscale, int M, int I, int K,
                                                                 int64_t sxm, const void* nwp, int nw_dtype,
                                                                 float eps) {
  typedef typename Vec8<T>::type V8;
  constexpr bool F8 = sizeof(W) == 1;
  constexpr DmaGeom G = dma_geom(sizeof(W));
  constexpr int NA = F8 ? 2 : 4;  // A reads per unit per lane
  constexpr int NT = NW * kWave;
  constexpr int TPR = NT / kResRows;  // threads per activation row in the prologue
  static_assert(TPR == 16 || TPR == 32 || TPR == 64, "two, four or eight waves");
  __shared__ u32x4 ring[NW][D][G.ae];
  extern __shared__ u32x4 dyn[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int r = lane & 15, g = lane >> 4;
  const int units = (K + kUnit - 1) / kUnit, kp = units * kUnit, cpr = kp / 8;
  const int tiles = I / 8;
  const int mine = (units - wave + NW - 1) / NW;  // >= 1: the host launches NW <= units
  const int ntw = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;  // 1..kResMaxTiles
  const int total = ntw * mine;                                                   // >= D
  u32x4* xs = dyn;                   // kResRows rows of cpr chunks
  u32x4* wl = dyn + kResRows * cpr;  // prologue: the norm weight, raw; then the partial sums
  u32x4* scl = wl + res_shared_bytes(kp, NW) / 16;  // E4M3: row scales, 16 floats per tile iteration
  const unsigned xs0 = lds_addr(xs), wl0 = lds_addr(wl), sc0 = lds_addr(scl);

  // ---- prologue DMAs: the rows, the norm weight, the row scales
  {
    const int per_row = cpr / kWave;  // instructions per row (cpr is a multiple of 64)
    for (int q = wave; q < kResRows * per_row; q += NW) {
      const int row = q / per_row, p = (q - row * per_row) * kWave + lane;
      const int c = p ^ (row & 7);
      dma16(x + (int64_t)(row < M ? row : 0) * sxm + (int64_t)c * 8, xs + row * cpr + (p - lane));
    }
    const int wb = nw_dtype == FD_F32 ? 4 : 2, epc = 16 / wb;
    const int wins = (kp * wb) / 16 / kWave;  // DMA instructions for the norm weight
    const char* wsrc = static_cast<const char*>(nwp);
    for (int q = wave; q < wins; q += NW) {
      const int64_t k = (int64_t)(q * kWave + lane) * epc;
      dma16(wsrc + k * wb, wl + q * kWave);
    }
    if constexpr (F8) {
      if (wave == 0) {
        const int i = lane >> 2, qq = lane & 3;
        const int t = (int)blockIdx.x + (i < ntw ? i : 0) * (int)gridDim.x;
        const int64_t row = qq < 2 ? (int64_t)8 * t + 4 * qq : (int64_t)I + 8 * t + 4 * (qq - 2);
        dma16(wscale + row, scl);
      }
    }
  }

  // ---- weight stream
  const unsigned ring0 = lds_addr(&ring[wave][0][0]);
  int wch[G.aops], wrw[G.aops];  // K offset of this lane's chunk; its tile row (0-15)
#pragma unroll
  for (int i = 0; i < G.aops; ++i) {
    const int row = G.rpi * i + lane / G.cpr;
    wrw[i] = row;
    wch[i] = ((lane % G.cpr) ^ (row % G.cpr)) * G.epc;
  }
  // this lane's chunk of the issue tile's rows at the wave's first unit; a unit
  // adds only its K offset (the row addresses change once per tile)
  const W* wb[G.aops];
  auto set_tile = [&](int itile) {
    const int t = (int)blockIdx.x + itile * (int)gridDim.x;
#pragma unroll
    for (int i = 0; i < G.aops; ++i) {
      const int row = wrw[i];
      const int64_t n = row < 8 ? (int64_t)8 * t + row : (int64_t)I + 8 * t + (row - 8);
      wb[i] = w + n * (int64_t)K + wave * kUnit + wch[i];
    }
  };
  set_tile(0);
  int it = 0, iu = 0, koff = 0;  // issue cursor: tile iteration, unit of this wave, its K offset
  auto issue = [&](int slot) {
    u32x4* dst = ring[wave][slot];
#pragma unroll
    for (int i = 0; i < G.aops; ++i) dma16_nt(wb[i] + koff, dst + i * kWave);
    koff += NW * kUnit;
    if (++iu == mine) {
      iu = 0;
      koff = 0;
      if (++it < ntw) set_tile(it);
    }
  };
#pragma unroll
  for (int u = 0; u < D; ++u) issue(u);

  // ---- normalise the resident rows (each thread: one row, chunks lane%TPR + TPR*i)
  wait_vm<G.aops * D>();  // this wave's prologue DMAs have landed (its D units may not have)
  res_barrier();          // ... and every wave's
  {
    const int row = tid / TPR, c0 = tid % TPR;
    const unsigned rb = xs0 + (unsigned)(row * cpr) * 16u;
    auto slot_of = [&](int c) { return rb + (unsigned)(c ^ (row & 7)) * 16u; };
    float ss = 0.f;
    for (int c = c0; c < cpr; c += 4 * TPR) {
      u32x4 v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = ds_read16(slot_of(c + i * TPR < cpr ? c + i * TPR : c));
      res_wait_lds(v);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c + i * TPR < cpr) ss = dot8(__builtin_bit_cast(V8, v[i]), __builtin_bit_cast(V8, v[i]), ss);
    }
    if constexpr (TPR >= 32) ss = xlane_sum<16>(ss);
    ss = xlane_sum<8>(ss);
    ss = xlane_sum<4>(ss);
    ss = xlane_sum<2>(ss);
    ss = xlane_sum<1>(ss);
    if constexpr (TPR == 64) ss = xlane_sum<32>(ss);
    const float inv = row < M ? rsqrtf(ss / (float)K + eps) : 0.f;
    const bool wf = nw_dtype == FD_F32;
    for (int c = c0; c < cpr; c += TPR) {
      u32x4 v[3];
      v[0] = ds_read16(slot_of(c));
      v[1] = ds_read16(wl0 + (unsigned)(wf ? 2 * c : c) * 16u);
      v[2] = ds_read16(wl0 + (unsigned)(wf ? 2 * c + 1 : c) * 16u);
      res_wait_lds(v);
      ds_write16(slot_of(c), wf ? norm_frag<T>(v[0], inv, v[1], v[2]) : norm_frag_w<T>(v[0], inv, v[1]));
    }
  }
  res_barrier();  // the rows are normalised

  // ---- main loop
  unsigned fa[NA];
#pragma unroll
  for (int t = 0; t < NA; ++t)
    fa[t] = F8 ? ring0 + (unsigned)(r * 8 + ((2 * g + t) ^ (r & 7))) * 16u
               : ring0 + (unsigned)(r * 16 + ((t * 4 + g) ^ r)) * 16u;
  const int hi = r >= 8, brow = half_b_row(r);  // half-B: fragments 2p + hi of row brow
  const unsigned xb = xs0 + (unsigned)(brow * cpr) * 16u;
  int ktl[2];  // chunk of fragment p within a unit
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int s2 = 2 * p + hi;
    ktl[p] = F8 ? 4 * g + s2 : 4 * s2 + g;
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int cu = 0, ct = 0;  // consume cursor
  for (int j = 0; j < total; ++j) {
    const int slot = j % D;
    if (j + D <= total)
      wait_vm<G.aops * (D - 1)>();
    else
      wait_vm<0>();
    {
      const unsigned so = (unsigned)slot * (G.ae * 16u);
      const int k0 = (wave + cu * NW) * kUnit;
      u32x4 v[NA + 2];
#pragma unroll
      for (int t = 0; t < NA; ++t) v[t] = ds_read16(fa[t] + so);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int c = k0 / 8 + ktl[p];
        v[NA + p] = ds_read16(xb + (unsigned)(c ^ (brow & 7)) * 16u);
      }
      res_wait_lds(v);
      u32x4 b[4];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        b[2 * p] = v[NA + p];
        b[2 * p + 1] = mirror16(b[2 * p]);
      }
      u32x4 af[4];
      if constexpr (F8) {
        fp8x16_decode<T>(v[0], af[0], af[1]);
        fp8x16_decode<T>(v[1], af[2], af[3]);
      } else {
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) af[s2] = v[s2];
      }
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2)
        acc = mfma16(__builtin_bit_cast(V8, af[s2]), __builtin_bit_cast(V8, b[s2]), acc);
    }
    if (j + D < total) issue(slot);
    if (++cu == mine) {  // this wave's last unit of tile iteration ct
      const unsigned pb = wl0 + (unsigned)((ct & 1) * NW * kWave) * 16u;  // the norm weight is done with
      ds_write16(pb + (unsigned)(wave * kWave + lane) * 16u, __builtin_bit_cast(u32x4, acc));
      acc = f32x4{0.f, 0.f, 0.f, 0.f};
      res_barrier();
      if (wave == ct % NW) {
        u32x4 pv[NW + 1];
#pragma unroll
        for (int i = 0; i < NW; ++i) pv[i] = ds_read16(pb + (unsigned)(i * kWave + lane) * 16u);
        const int nb = (lane >> 4) * 4;
        pv[NW] = ds_read16(sc0 + (unsigned)(ct * 16 + nb) * 4u);  // E4M3 row scales (unused otherwise)
        res_wait_lds(pv);
        f32x4 s = __builtin_bit_cast(f32x4, pv[0]);
#pragma unroll
        for (int i = 1; i < NW; ++i) s += __builtin_bit_cast(f32x4, pv[i]);
        if constexpr (F8) s *= __builtin_bit_cast(f32x4, pv[NW]);
        const int t = (int)blockIdx.x + ct * (int)gridDim.x, m = lane & 15;
        float u[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) u[i] = xlane_partner32(s[i], lane);
        if (nb < 8 && m < M) {
#pragma unroll
          for (int i = 0; i < 4; ++i) mid[(int64_t)m * I + 8 * t + nb + i] = swiglu_out<T>(s[i], u[i]);
        }
      }
      cu = 0;
      ++ct;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side

inline int res_grid(int I) {
  const int tiles = I / 8, cus = device_cus();
  return tiles < cus ? tiles : cus;
}

// Whether the persistent form takes a gate/up: 5-8 rows; K a multiple of 512
// (one DMA instruction covers 64 chunks of a row, and no unit crosses K), at
// least D units per wave and tile; whole 16-row tiles that one workgroup per CU
// covers in at most kResMaxTiles iterations; a float32 norm weight or one in
// the activations' type; the LDS of one CU.
template <typename T, typename W, int NW, int D>
inline bool res_takes(int64_t M, int64_t I, int64_t K, int nw_dtype) {
  if (M < 5 || M > kResRows || I % 8 != 0 || I < 8 || K % 512 != 0 || (K / kUnit) / NW < D) return false;
  if (nw_dtype != FD_F32 && nw_dtype != (std::is_same<T, f16>::value ? FD_F16 : FD_BF16)) return false;
  const int tiles = (int)(I / 8), grid = res_grid((int)I);
  if ((tiles + grid - 1) / grid > kResMaxTiles) return false;
  return res_static_lds(NW, D, sizeof(W)) + res_dyn_lds((int)K, NW) <= kMaxLds;
}

template <typename T, typename W, int NW, int D>
int launch_gate_up_res(void* mid, const void* x, const W* w, const float* wscale, int M, int I, int K,
                       int64_t sxm, const void* nw, int nw_dtype, float eps, hipStream_t st) {
  auto kernel = gate_up_res_kernel<T, W, NW, D>;
  const size_t dyn = res_dyn_lds(K, NW);
  if (!allow_lds(kernel, dyn)) return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", dyn);
  hipLaunchKernelGGL(kernel, dim3((unsigned)res_grid(I)), dim3(NW * kWave), dyn, st, static_cast<T*>(mid),
                     static_cast<const T*>(x), w, wscale, M, I, K, sxm, nw, nw_dtype, eps);
  return FD_OK;
}

}  // namespace fd
