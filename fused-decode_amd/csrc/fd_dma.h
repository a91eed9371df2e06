// MFMA GEMV for 5-16 activation rows with its tiles streamed into LDS by DMA,
// shared by the fp16/bf16 and the E4M3 entry points.
//
// A workgroup of NW waves owns 16 weight rows; wave w takes K units w, w + NW,
// ... of a sweep that starts at the workgroup's XCD offset (sweep_unit). A unit
// is 128 K elements: the 16-row weight tile (4 KiB of fp16/bf16, 2 KiB of E4M3
// codes) and the BR-row activation tile (BR = M rounded up to 4, 8 or 16),
// moved by global_load_lds_dwordx4 instructions (nontemporal for the weights,
// which are read once; cached for the activations, which every workgroup
// re-reads) into one of the wave's D ring
// slots, D units in flight. Lane L of an instruction
// fills ring entry 16*L of it; the lane picks its source chunk so that the slot
// holds every row XOR-swizzled (chunk c of row r at position c ^ (r mod
// chunks-per-row)), which keeps the fragment reads of 8 lanes on distinct bank
// groups. Activation rows past M re-read row 0 and weight rows past N row 0
// (their outputs are never stored). In a unit that crosses K, lanes fetch their
// row's first chunk for chunks past K and then overwrite those ring entries
// with zeros, so every unit runs the same four v_mfma_f32_16x16x32 steps.
//
// k order inside a unit. fp16/bf16 weights: MFMA step s takes k = 32 s + 8 g +
// j for the lane of k-group g (element j of its fragment), so a lane reads
// chunk 4 s + g of its row. E4M3 weights: step s takes k = 32 g + 8 s + j, so a
// lane's four fragments are its row's 32 consecutive codes (two 16-byte reads,
// decoded exactly to the activation type by v_cvt_scalef32_pk_*_fp8), and its
// B fragments the matching activations (chunk 4 g + s). Any k order that A and
// B share gives the same sum of products.
//
// Epilogues. EPI_PLAIN: tile rows n0..n0+15, bias / row_add / rounding as the
// GEMV. EPI_ROPE (fused QKV): rows placed by TileRows<16>, rotated tiles rotate
// their rounded outputs (cos/sin staged through LDS, see angle_loads). E4M3 sums are
// multiplied by the row's channel scale first.
//
// With NORM, x is the raw activation and the kernel applies the RMSNorm itself.
// A prologue whose loads go out just before the first units' DMAs derives the
// rows' inverse RMS, from x or from the producer's row sums (with those and a
// streamed weight, in every wave, with no workgroup barrier). The norm weight
// streams with the units when it has the activations' dtype (NORM_STREAMED), or
// the prologue stages it in dynamic LDS as float32 (NORM_STAGED, norm_dma_lds
// bytes). Every B fragment is normalised after its LDS read (up to 8 rows in the
// half-B form: each lane normalises two fragments and swaps them with its
// row-mirror partner).
#pragma once

#include "fd_gemv.h"

namespace fd {

enum DmaEpi { EPI_PLAIN = 0, EPI_ROPE = 1 };

// How a launch applies the folded RMSNorm: not at all; with the norm weight
// staged in LDS as float32 by the prologue (any weight dtype); or with the
// weight (in the activation type) streamed with each unit like the activations,
// so the prologue waits only for the row sums.
enum DmaNorm { NORM_NONE = 0, NORM_STAGED = 1, NORM_STREAMED = 2 };

// Ring geometry of one unit's 16-row weight tile for weights of `bytes` bytes.
struct DmaGeom {
  int cpr;   // 16-byte chunks per 128-element row: 16 or 8
  int epc;   // weight elements per chunk: 8 or 16
  int ae;    // ring entries of the tile: 256 or 128
  int aops;  // its DMA instructions: 4 or 2
  int rpi;   // rows per instruction: 4 or 8
};
__host__ __device__ constexpr DmaGeom dma_geom(int bytes) {
  return DmaGeom{kUnit * bytes / 16, 16 / bytes, 16 * (kUnit * bytes / 16), 16 * (kUnit * bytes / 16) / kWave,
                 kWave / (kUnit * bytes / 16)};
}

// Static LDS of a DMA launch: the ring (NW waves x D slots of the weight tile,
// the B rows and, streaming the norm weight, its 16 entries) and the partial
// sums.
__host__ __device__ constexpr size_t dma_lds(int nw, int d, int br, int wbytes = 2, bool ws = false) {
  return (size_t)nw * d * (dma_geom(wbytes).ae + br * 16 + (ws ? 16 : 0)) * 16 + (size_t)nw * kWave * 16;
}

// Dynamic LDS of a NORM launch: NORM_STAGED the float32 norm weight over whole
// K units; both modes the 16 inverse RMS values and the prologue's reduction
// scratch.
inline size_t norm_dma_lds(int K, int mode) {
  const size_t w = mode == NORM_STAGED ? (size_t)((K + kUnit - 1) / kUnit) * kUnit : 0;
  return sizeof(float) * (w + 16 + kMaxWaves * 16);
}

// Activation rows a DMA MFMA launch stages: M rounded up to 4, 8 or 16.
inline int dma_rows(int M) { return M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// Make the NR ds_read16 results in `v` usable: one s_waitcnt lgkmcnt(0) that
// names every register, so no use is scheduled ahead of it.
#define FD_V1(i) "+v"(v[i])
#define FD_V6 FD_V1(0), FD_V1(1), FD_V1(2), FD_V1(3), FD_V1(4), FD_V1(5)
#define FD_V8 FD_V6, FD_V1(6), FD_V1(7)
#define FD_V10 FD_V8, FD_V1(8), FD_V1(9)
#define FD_V12 FD_V10, FD_V1(10), FD_V1(11)
#define FD_V14 FD_V12, FD_V1(12), FD_V1(13)
#define FD_V16 FD_V14, FD_V1(14), FD_V1(15)
template <int NR>
__device__ __forceinline__ void wait_lds_all(u32x4 (&v)[NR]) {
  if constexpr (NR == 6)
    asm volatile("s_waitcnt lgkmcnt(0)" : FD_V6::"memory");
  else if constexpr (NR == 8)
    asm volatile("s_waitcnt lgkmcnt(0)" : FD_V8::"memory");
  else if constexpr (NR == 10)
    asm volatile("s_waitcnt lgkmcnt(0)" : FD_V10::"memory");
  else if constexpr (NR == 12)
    asm volatile("s_waitcnt lgkmcnt(0)" : FD_V12::"memory");
  else if constexpr (NR == 14)
    asm volatile("s_waitcnt lgkmcnt(0)" : FD_V14::"memory");
  else if constexpr (NR == 16)
    asm volatile("s_waitcnt lgkmcnt(0)" : FD_V16::"memory");
  else
    static_assert(NR == 6, "no register list for this fragment count");
}
template <int N1, int N2>
__device__ __forceinline__ void wait_lds_all(u32x4 (&a)[N1], u32x4 (&b)[N2]) {
  if constexpr (N1 == 2 && N2 == 4)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3])::"memory");
  else if constexpr (N1 == 1 && N2 == 2)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(b[0]), "+v"(b[1])::"memory");
  else
    static_assert(N1 == 2 && N2 == 4, "no register list for these counts");
}
#undef FD_V1
#undef FD_V6
#undef FD_V8
#undef FD_V10
#undef FD_V12
#undef FD_V14
#undef FD_V16

// Sixteen E4M3 codes (byte 0 first) -> two 8-element fragments of their exact
// values in T.
template <typename T>
__device__ __forceinline__ void fp8x16_decode(const u32x4& w, u32x4& c0, u32x4& c1) {
  uint32_t h[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (std::is_same<T, f16>::value) {
      h[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[i], 1.0f, false));
      h[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[i], 1.0f, true));
    } else {
      h[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, false));
      h[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, true));
    }
  }
  c0 = u32x4{h[0], h[1], h[2], h[3]};
  c1 = u32x4{h[4], h[5], h[6], h[7]};
}

template <typename T, typename W, int NW, int D, int BR, int EPI, int NORM>
__global__ __launch_bounds__(NW * kWave) void gemv_mfma_dma_kernel(
    T* y, const T* x, const W* w, const float* wscale, int M, int N, int K, int64_t sxm,
    int64_t swn, int64_t sym, int64_t syn, Epi e, Rope rp, const void* nwp, int nw_dtype,
    float eps, RowSq rq) {
  typedef typename Vec8<T>::type V8;
  constexpr bool F8 = sizeof(W) == 1;
  constexpr DmaGeom G = dma_geom(sizeof(W));
  constexpr int NA = F8 ? 2 : 4;               // A reads per unit per lane
  // NORM up to 8 rows: the half-B form (half_b_row / mirror16): a lane reads and
  // normalises two B fragments, steps 2p + hi, and the row mirror hands each
  // low lane its partner's; from 9 rows a lane normalises all four it reads
  constexpr bool NHALF = NORM && BR <= 8;
  constexpr bool WS = NORM == NORM_STREAMED;
  constexpr int NB = NHALF ? 2 : 4;                                    // B fragment reads per unit
  constexpr int NWR = NORM == NORM_STAGED ? 2 * NB : WS ? NB : 0;      // norm-weight reads per unit
  constexpr int NR = NA + NB + NWR;                                    // LDS reads per unit
  // 16-byte entries: the A tile, the B rows, WS: the unit's 128 norm weights
  // (16 entries, filled by lanes 0-15 of one DMA instruction)
  constexpr int WOFF = G.ae + BR * 16;
  constexpr int SLOT = WOFF + (WS ? 16 : 0);
  constexpr int OPS = G.aops + BR / 4 + (WS ? 1 : 0);  // DMA instructions per unit
  __shared__ u32x4 ring[NW][D][SLOT];
  __shared__ f32x4 part[NW * kWave];
  __shared__ float ang_lds[EPI == EPI_ROPE ? kTileAngles : 1];  // ROPE: the tile's cos/sin
  extern __shared__ float norm_lds[];  // NORM_STAGED: w [units * 128]; NORM: inv [16], scratch
  const int lane = threadIdx.x & (kWave - 1);
  // wave-uniform, so the unit indices, the K-tail tests and the ring addresses
  // are scalar (a per-lane value here turns the tail test into exec-masked
  // branches that shuttle the accumulator out of the MFMA registers every unit)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const TileRows<16> tr(rp, EPI == EPI_ROPE ? (int)blockIdx.x : 0);
  const W* wrow[G.aops];
  int wch[G.aops];  // K offset (elements) of this lane's chunk in instruction i
#pragma unroll
  for (int i = 0; i < G.aops; ++i) {
    const int row = G.rpi * i + lane / G.cpr;
    const int64_t n = EPI == EPI_ROPE ? tr.row(row) : n0 + row;
    wrow[i] = w + (n < N ? n : 0) * swn;
    wch[i] = ((lane % G.cpr) ^ (row % G.cpr)) * G.epc;
  }
  const T* xrow[BR / 4];
  int xch[BR / 4];
#pragma unroll
  for (int i = 0; i < BR / 4; ++i) {
    const int row = 4 * i + (lane >> 4);
    xrow[i] = x + (row < M ? row : 0) * sxm;
    xch[i] = ((lane & 15) ^ row) * 8;
  }
  const int units = (K + kUnit - 1) / kUnit;
  const int mine = wave < units ? (units - wave + NW - 1) / NW : 0;
  const int off = sweep_offset(units);
  const T* nwt = static_cast<const T*>(nwp);  // WS: the norm weight, in T
  const int wsc = (lane & 15) * 8;            // WS: this lane's chunk of a unit's norm weights
  auto issue = [&](int j) {
    const int k0 = sweep_unit(wave, j, NW, off, units) * kUnit;
    u32x4* slot = ring[wave][j % D];
    if (k0 + kUnit <= K) {  // a whole unit (every unit but a K tail): no clamps
#pragma unroll
      for (int i = 0; i < G.aops; ++i) dma16_nt(wrow[i] + k0 + wch[i], slot + i * kWave);
#pragma unroll
      for (int i = 0; i < BR / 4; ++i) dma16(xrow[i] + k0 + xch[i], slot + G.ae + i * kWave);
      if constexpr (WS)
        if (lane < 16) dma16(nwt + k0 + wsc, slot + WOFF);
    } else {  // the same instruction count, chunks past K clamped to the row's first
#pragma unroll
      for (int i = 0; i < G.aops; ++i) {
        const int k = k0 + wch[i];
        dma16_nt(wrow[i] + (k < K ? k : 0), slot + i * kWave);
      }
#pragma unroll
      for (int i = 0; i < BR / 4; ++i) {
        const int k = k0 + xch[i];
        dma16(xrow[i] + (k < K ? k : 0), slot + G.ae + i * kWave);
      }
      if constexpr (WS) {
        const int k = k0 + wsc;
        if (lane < 16) dma16(nwt + (k < K ? k : 0), slot + WOFF);
      }
    }
  };
  // this lane's fragment entries within a slot (bytes)
  const unsigned ring0 = lds_addr(&ring[wave][0][0]);
  const int rb = r % BR;
  unsigned fa[NA], fb[4];
#pragma unroll
  for (int t = 0; t < NA; ++t)
    fa[t] = F8 ? ring0 + (unsigned)(r * 8 + ((2 * g + t) ^ (r & 7))) * 16u
               : ring0 + (unsigned)(r * 16 + ((t * 4 + g) ^ r)) * 16u;
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) {
    const int cb = F8 ? g * 4 + s2 : s2 * 4 + g;
    fb[s2] = ring0 + (unsigned)(G.ae + rb * 16 + (cb ^ rb)) * 16u;
  }
  const int hi = r >= 8, hrow = half_b_row(r) % BR;  // NHALF: this lane's B row
  if constexpr (NHALF) {  // fb[p]: fragment 2p + hi of row hrow
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int s2 = 2 * p + hi, cb = F8 ? g * 4 + s2 : s2 * 4 + g;
      fb[p] = ring0 + (unsigned)(G.ae + hrow * 16 + (cb ^ hrow)) * 16u;
    }
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float rinv = 0.f;       // NORM: inverse RMS of this lane's B row
  unsigned fwl = 0;       // NORM_STAGED: the staged norm weight (bytes)
  auto consume = [&](int j) {
    const unsigned so = (unsigned)(j % D) * (SLOT * 16u);
    const int k0 = sweep_unit(wave, j, NW, off, units) * kUnit;
    if (k0 + kUnit > K) {  // K tail: zero the entries fetched past K
#pragma unroll
      for (int i = 0; i < G.aops; ++i)
        if (k0 + wch[i] >= K) ds_zero16(ring0 + so + (unsigned)(i * kWave + lane) * 16u);
#pragma unroll
      for (int i = 0; i < BR / 4; ++i)
        if (k0 + xch[i] >= K) ds_zero16(ring0 + so + (unsigned)(G.ae + i * kWave + lane) * 16u);
      if constexpr (WS)
        if (lane < 16 && k0 + wsc >= K) ds_zero16(ring0 + so + (unsigned)(WOFF + lane) * 16u);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // v: [NA] A reads, [NB] B fragments, then the norm weight at their k:
    // NORM_STAGED 8 floats each (two reads), WS 8 T values each (one read)
    u32x4 v[NR];
#pragma unroll
    for (int t = 0; t < NA; ++t) v[t] = ds_read16(fa[t] + so);
#pragma unroll
    for (int t = 0; t < NB; ++t) v[NA + t] = ds_read16(fb[t] + so);
    if constexpr (NORM) {
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        const int s2 = NHALF ? 2 * t + hi : t;
        const int kl = F8 ? 32 * g + 8 * s2 : 32 * s2 + 8 * g;  // fragment t's first k in the unit
        if constexpr (WS) {
          v[NA + NB + t] = ds_read16(ring0 + so + (unsigned)(WOFF + kl / 8) * 16u);
        } else {
          const unsigned wa = fwl + (unsigned)(k0 + kl) * 4u;
          v[NA + NB + 2 * t] = ds_read16(wa);
          v[NA + NB + 2 * t + 1] = ds_read16(wa + 16u);
        }
      }
    }
    wait_lds_all(v);
    auto normed = [&](int t) {
      if constexpr (WS)
        return norm_frag_w<T>(v[NA + t], rinv, v[NA + NB + t]);
      else
        return norm_frag<T>(v[NA + t], rinv, v[NA + NB + 2 * t], v[NA + NB + 2 * t + 1]);
    };
    u32x4 b[4];
    if constexpr (NHALF) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        b[2 * p] = normed(p);
        b[2 * p + 1] = mirror16(b[2 * p]);
      }
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        if constexpr (NORM)
          b[s2] = normed(s2);
        else
          b[s2] = v[NA + s2];
      }
    }
    u32x4 af[4];
    if constexpr (F8) {
      fp8x16_decode<T>(v[0], af[0], af[1]);
      fp8x16_decode<T>(v[1], af[2], af[3]);
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) af[s2] = v[s2 & (NA - 1)];
    }
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
      acc = mfma16(__builtin_bit_cast(V8, af[s2]), __builtin_bit_cast(V8, b[s2]), acc);
  };
  const int pre = mine < D ? mine : D;
  // wave 0 writes the tile: its cos/sin loads go out first, so they complete
  // under the main loop's first wait instead of after the loop
  constexpr int APER = (kTileAngles + NW * kWave - 1) / (NW * kWave);
  AngleLoads<APER> ang{};
  if constexpr (EPI == EPI_ROPE) ang = angle_loads<APER>(rp, tr, M, wrow[0]);
  TileEpi tep{};
  if constexpr (EPI == EPI_PLAIN) tep = tile_epi_loads<F8>(e, wscale, wrow[0], lane, n0, M, N);
  bool wave_sums = false;
  if constexpr (WS && !F8) wave_sums = rq.p != nullptr;
  if (wave_sums) {
    // streamed norm weight and the producer's row sums: each wave adds all the
    // tiles' sums itself (its lanes take tiles lane, lane + 64, ...), so no
    // workgroup barrier stands between the sums and the first unit (fp16/bf16
    // weights, QKV at M=8: 14.0 -> 13.7 us; with E4M3 weights, whose units
    // arrive twice as fast, the four waves' extra reads of the sums cost more:
    // 11.5 -> 11.7 us, so those keep the workgroup prologue)
    constexpr int MP = pow2_ceil(BR), MQ = BR / 4, TQ = 4;
    float ss[MP];
#pragma unroll
    for (int m = 0; m < MP; ++m) ss[m] = 0.f;
    f32x4 q[TQ][MQ];
    auto tile_rows = [&](int t, f32x4 (&d)[MQ]) {
      const f32x4* src = reinterpret_cast<const f32x4*>(rq.p + (int64_t)(t < rq.parts ? t : 0) * 16);
#pragma unroll
      for (int i = 0; i < MQ; ++i) d[i] = src[i];
    };
    auto add_tile = [&](const f32x4 (&d)[MQ]) {
#pragma unroll
      for (int m = 0; m < BR; ++m) ss[m] += d[m / 4][m % 4];
    };
#pragma unroll
    for (int i = 0; i < TQ; ++i) tile_rows(lane + i * kWave, q[i]);
    for (int j = 0; j < pre; ++j) issue(j);  // behind the sums' loads, which complete first
#pragma unroll
    for (int i = 0; i < TQ; ++i)
      if (lane + i * kWave < rq.parts) add_tile(q[i]);
    for (int t = lane + TQ * kWave; t < rq.parts; t += kWave) {
      tile_rows(t, q[0]);
      add_tile(q[0]);
    }
    butterfly_sum<MP>(ss, lane);  // lane l: the sum of row butterfly_index<MP>(l)
    const int row = butterfly_index<MP>(lane);
    const float il = row < M ? rsqrtf(ss[0] / (float)K + eps) : 0.f;
    const int want = (NHALF ? hrow : rb) * (kWave / MP);  // a lane holding this lane's row
    rinv = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(want << 2, __builtin_bit_cast(int, il)));
  } else if constexpr (NORM) {
    float* wl = norm_lds;
    float* inv = norm_lds + (WS ? 0 : units * kUnit);
    norm_prologue<T, BR, true, NW * kWave, !WS>(wl, inv, inv + 16, nwp, nw_dtype, x, sxm, M, K, units * kUnit, eps,
                                                rq, [&] {
                                                  for (int j = 0; j < pre; ++j) issue(j);
                                                });
    rinv = inv[NHALF ? hrow : rb];
    fwl = lds_addr(wl);
  } else {
    for (int j = 0; j < pre; ++j) issue(j);
  }
  int j = 0;
  for (; j + D <= mine; ++j) {  // D units in flight: the D-1 after unit j may stay outstanding
    wait_vm<OPS * (D - 1)>();
    consume(j);
    if (j + D < mine) issue(j + D);
  }
  wait_vm<0>();
  for (; j < mine; ++j) consume(j);
  if constexpr (EPI == EPI_ROPE) angle_store<APER>(ang_lds, ang, rp, tr, M);
  part[wave * kWave + lane] = acc;
  __syncthreads();
  if (threadIdx.x < kWave) {
    f32x4 s = part[threadIdx.x];
    for (int i = 1; i < NW; ++i) s += part[i * kWave + threadIdx.x];
    if constexpr (EPI == EPI_PLAIN)
      mfma_tile_out_plain<T, F8>(y, s, threadIdx.x, n0, e, tep, M, N, sym, syn);
    else if constexpr (F8)
      mfma_tile_out<T, true>(y, s, threadIdx.x, n0, tr, e, ang_lds, rp.rs, RowScale{wscale}, M, N, sym, syn);
    else
      mfma_tile_out<T, true>(y, s, threadIdx.x, n0, tr, e, ang_lds, rp.rs, NoScale{}, M, N, sym, syn);
  }
}

// ---------------------------------------------------------------------------
// Host side

// The RMSNorm folded into a DMA MFMA launch (x = raw activations, normalised in
// the kernel with norm_w / eps).
struct FoldNorm {
  const void* w;
  int dtype;
  float eps;
  RowSq sq = {nullptr, 0};  // the producer's row sums of squares of x, if it wrote them
};

template <typename T, typename W, int NW, int D, int BR, int EPI, int MODE>
int launch_dma_mode(unsigned blocks, void* y, const void* x, const void* w, const float* ws, int M,
                    int N, int K, int64_t sxm, int64_t swn, int64_t sym, int64_t syn, const Epi& e,
                    const Rope& r, const FoldNorm& fn, hipStream_t st) {
  constexpr size_t lds = dma_lds(NW, D, BR, sizeof(W), MODE == NORM_STREAMED) +
                         (EPI == EPI_ROPE ? kTileAngles * sizeof(float) : 0);
  if constexpr (lds <= kMaxLds) {
    const size_t dyn = MODE ? norm_dma_lds(K, MODE) : 0;
    auto kernel = gemv_mfma_dma_kernel<T, W, NW, D, BR, EPI, MODE>;
    if (lds + dyn > kMaxLds)
      return set_error(FD_EUNSUPPORTED, "K too large for the folded RMSNorm's LDS stage");
    if (!allow_lds(kernel, dyn))
      return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", dyn);
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(NW * kWave), dyn, st, static_cast<T*>(y),
                       static_cast<const T*>(x), static_cast<const W*>(w), ws, M, N, K, sxm, swn,
                       sym, syn, e, r, fn.w, fn.dtype, fn.eps, fn.sq);
    return FD_OK;
  }
  return set_error(FD_EINVAL, "MFMA tile beyond the LDS of a CU");
}

// NORM: the norm weight streams with the units when it has the activations'
// dtype (one 16-byte read per B fragment, nothing staged before the first unit),
// else the prologue stages it as float32.
template <typename T, typename W, int NW, int D, int BR, int EPI, bool NORM>
int launch_dma(unsigned blocks, void* y, const void* x, const void* w, const float* ws, int M,
               int N, int K, int64_t sxm, int64_t swn, int64_t sym, int64_t syn, const Epi& e,
               const Rope& r, const FoldNorm& fn, hipStream_t st) {
  if constexpr (NORM) {
    if (fn.dtype == (std::is_same<T, f16>::value ? FD_F16 : FD_BF16))
      return launch_dma_mode<T, W, NW, D, BR, EPI, NORM_STREAMED>(blocks, y, x, w, ws, M, N, K, sxm, swn, sym,
                                                                  syn, e, r, fn, st);
    return launch_dma_mode<T, W, NW, D, BR, EPI, NORM_STAGED>(blocks, y, x, w, ws, M, N, K, sxm, swn, sym, syn,
                                                              e, r, fn, st);
  }
  return launch_dma_mode<T, W, NW, D, BR, EPI, NORM_NONE>(blocks, y, x, w, ws, M, N, K, sxm, swn, sym, syn, e, r,
                                                          fn, st);
}

template <typename T, typename W, int NW, int D, int EPI, bool NORM>
int launch_dma_rows(unsigned blocks, void* y, const void* x, const void* w, const float* ws, int M,
                    int N, int K, int64_t sxm, int64_t swn, int64_t sym, int64_t syn, const Epi& e,
                    const Rope& r, const FoldNorm& fn, hipStream_t st) {
  const int br = dma_rows(M);
  if (br == 4)
    return launch_dma<T, W, NW, D, 4, EPI, NORM>(blocks, y, x, w, ws, M, N, K, sxm, swn, sym, syn, e, r, fn, st);
  if (br == 8)
    return launch_dma<T, W, NW, D, 8, EPI, NORM>(blocks, y, x, w, ws, M, N, K, sxm, swn, sym, syn, e, r, fn, st);
  return launch_dma<T, W, NW, D, 16, EPI, NORM>(blocks, y, x, w, ws, M, N, K, sxm, swn, sym, syn, e, r, fn, st);
}

// The default launch shape: four waves (two when K has fewer than four units),
// two units in flight each.
template <typename T, typename W, int EPI, bool NORM>
int launch_dma_default(unsigned blocks, void* y, const void* x, const void* w, const float* ws,
                       int M, int N, int K, int64_t sxm, int64_t swn, int64_t sym, int64_t syn,
                       const Epi& e, const Rope& r, const FoldNorm& fn, hipStream_t st) {
  if ((K + kUnit - 1) / kUnit >= 4)
    return launch_dma_rows<T, W, 4, 2, EPI, NORM>(blocks, y, x, w, ws, M, N, K, sxm, swn, sym, syn, e, r, fn, st);
  return launch_dma_rows<T, W, 2, 2, EPI, NORM>(blocks, y, x, w, ws, M, N, K, sxm, swn, sym, syn, e, r, fn, st);
}

}  // namespace fd
