// Small-M GEMV (M <= 16) and the fused Llama post-attention MLP for gfx950.
//
//   y[m,n] = round(sum_k x[m,k] * w[n,k] + bias[n] + row_add[m,n])
//
// At M <= 16 the product is weight streaming: every weight byte is read once
// from HBM and used for M multiply-adds, so the kernels are built to keep many
// 16-byte weight loads in flight and to touch every 128-byte line whole.
//
// SIMT kernel (gemv_simt_kernel, exact M): a workgroup owns R weight rows; its
// waves split K into 512-element chunks (64 lanes x one 16-byte vector), each
// lane streams its vector of every row and folds it against x with v_dot2
// (fp16/bf16 pairs into float32). Per-lane partial sums are combined with a
// transposing butterfly (V-1 exchanges for V sums) and then across waves in LDS.
//
// MFMA kernel (gemv_mfma_relayout_kernel, M padded to 16; kind=dot from 5 rows):
// a workgroup owns 16 weight rows; waves split K into 128-element units of four
// v_mfma_f32_16x16x32 steps. A = 16 weight rows x 32 k (lane l: row l%16,
// k-group l/16), B = x^T with the same lane->k mapping; padding rows m >= M load
// row 0 again (their output columns are never stored). The weights are loaded
// row-contiguously and relaid through LDS into the A layout (see the kernel).
//
// Every hot loop issues its loads unconditionally (out-of-range lanes read an
// in-bounds address and are masked where used) and runs its K steps through
// two register buffers (stream_steps, fd_gemv.h), so a wave always has its next
// step's loads in flight; a guarded load would make the compiler wait for all
// outstanding loads at its first use.
//
// Fused MLP: launch 1 computes the RMSNorm of hidden in a prologue (each
// workgroup re-derives the row scale and stages the normalised activations in
// LDS), streams matching gate row j and up row I+j, and writes only
// mid = round(silu(round(g)) * round(u)). Launch 2 is the down GEMV with the
// residual fused as row_add. Weights are read once; gate_up never exists in HBM.
// From 5 rows (kind=dot) both launches use the MFMA form; up to 8 rows the
// gate/up kernel still normalises x itself, from 9 a row kernel writes the
// normalised rows first.
//
// Fused QKV (qkv_simt_kernel, and the MFMA kernel with ROPE): the same prologue
// and weight stream with tiles placed so that both halves of every rotate-half
// pair land in one workgroup, which applies RoPE in the epilogue.
#include <mutex>
#include <type_traits>

#include "fd_dma.h"
#include "fd_gemv.h"
#include "fd_internal.h"

namespace fd {

// Rows of the weight tile per SIMT workgroup for exact M (per-lane accumulators
// are R*M floats).
template <int M> struct SimtRows { static constexpr int R = 4; };
// The persistent SIMT GEMV with one K chunk per lane: four rows up to M = 4, two
// from 5, where the 8*M-float sums and their butterfly per tile cost the most
// (Llama-3-8B shapes, M = 8 / 16: N = K = 4096 9.18 / 12.97 us with two rows
// against 9.18 / 14.78 with four; N = 6144 11.89 / 17.40 against 12.30 / 19.79);
// with more chunks per lane simt_px_rows decides.
template <int M> struct SimtPxRows { static constexpr int R = M <= 4 ? 4 : 2; };
// Fused gate/up: R gate rows + R up rows.
template <int M> struct MlpRows { static constexpr int R = M <= 4 ? 4 : 2; };
// Fused QKV: R rows per tile (R/2 rotate-half pairs in a rotated tile); eight
// up to 2 rows (Llama-3-8B widths, M=1: 11.1 against 11.7 us for four).
template <int M> struct QkvRows { static constexpr int R = M <= 2 ? 8 : 4; };

// ---------------------------------------------------------------------------
// SIMT GEMV

template <typename T, int M, int R>
struct StepRegs {
  typename Vec8<T>::type w[R], x[M];
};

// At M = 1 a wave's K steps run through stream_steps with unconditional loads
// (a lane past K reads chunk 0, masked in the math), so the next step's weights
// and activations are in flight during the current step's math (1-3% faster on
// the decode shapes); from 2 rows the doubled registers cost more occupancy
// than the pipeline gains (M = 4, N = 28672: 47 against 39 us).
template <typename T, int M, int R, bool NTW>
__global__ __launch_bounds__(kMaxWaves * kWave) void gemv_simt_kernel(
    T* y, const T* x, const T* w, int N, int K, int64_t sxm, int64_t swn, int64_t sym,
    int64_t syn, Epi e) {
  typedef typename Vec8<T>::type V8;
  constexpr int V = pow2_ceil(R * M);
  __shared__ float part[kMaxWaves * V];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = block_threads() / kWave;
  const int64_t n0 = (int64_t)blockIdx.x * R;

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  const T* wr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wr[r] = w + (n0 + r < N ? n0 + r : 0) * swn;  // rows past N: never stored
  const int kbase = (wave * kWave + lane) * 8;
  const int step = nw * kChunk;

  if constexpr (M == 1) {
    auto issue = [&](StepRegs<T, M, R>& q, int s) {
      const int k = kbase + s * step;
      const int kc = k < K ? k : 0;
#pragma unroll
      for (int r = 0; r < R; ++r) q.w[r] = load8w<NTW, T>(wr[r] + kc);
#pragma unroll
      for (int m = 0; m < M; ++m) q.x[m] = load8<T>(x + m * sxm + kc);
    };
    auto consume = [&](const StepRegs<T, M, R>& q, int s) {
      if (kbase + s * step >= K) return;
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r * M + m] = dot8(q.w[r], q.x[m], acc[r * M + m]);
    };
    StepRegs<T, M, R> qa, qb;
    const int steps = (K + step - 1) / step;
    if (steps > 0) issue(qa, 0);  // K = 0 loads nothing (x may be null)
    stream_steps(steps, qa, qb, issue, consume);
  } else {
    for (int k = kbase; k < K; k += step) {
      V8 wv[R];
#pragma unroll
      for (int r = 0; r < R; ++r) wv[r] = load8w<NTW, T>(wr[r] + k);
      V8 xv[M];
#pragma unroll
      for (int m = 0; m < M; ++m) xv[m] = load8<T>(x + m * sxm + k);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r * M + m] = dot8(wv[r], xv[m], acc[r * M + m]);
    }
  }

  butterfly_sum<V>(acc, lane);
  if (butterfly_writer<V>(lane)) part[wave * V + butterfly_index<V>(lane)] = acc[0];
  __syncthreads();
  for (int t = threadIdx.x; t < R * M; t += block_threads()) {
    const int r = t / M, m = t % M;
    const int64_t n = n0 + r;
    if (n < N) {
      float s = 0.f;
      for (int i = 0; i < nw; ++i) s += part[i * V + t];
      y[m * sym + n * syn] = from_f32<T>(epilogue(e, s, m, n));
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent SIMT GEMV with the activations held in registers (exact M from 2
// rows, K up to CPL 512-element chunks per lane and eight waves)
//
// gemv_simt_kernel re-reads a wave's M activation vectors for every tile it
// works on and, with one K chunk per wave at K = 4096, waits out one memory
// latency per tile before a workgroup barrier. Here each wave owns CPL K chunks
// (1, 2 or 4: chunks wave, wave + nw, ...) for the whole launch: it loads its
// CPL * M activation vectors once, then walks the
// workgroup's weight tiles (blockIdx.x, + gridDim.x, ...; R rows each) with the
// next tile's rows in flight during this tile's math (stream_steps). After each
// tile the wave folds its R*M sums across its lanes (butterfly_sum) and parks
// them in LDS; one barrier after the last tile, then the workgroup adds the
// waves' sums of every tile it owns and writes the outputs. No barrier stands
// between tiles, so a wave whose loads arrive late delays no other. More chunks
// per lane spread the per-tile butterfly over more products (the activations'
// registers grow by M * 4 per chunk) and let K = 14336 run on seven waves.
//
// PH (K past what eight waves hold at CPL chunks per lane, e.g. 9-16 rows at
// K = 14336): the K chunks split into `phases` runs of nw * CPL; the wave walks
// its tiles once per phase (phase p: chunks p * nw * CPL + wave + c * nw) with
// that phase's activation vectors in its registers, and adds each tile's folded
// sums into its LDS slot: the activations are read once per phase per
// workgroup instead of once per tile, at the cost of one exposed load latency
// per phase (the registers hold one phase's activations, not two).
__host__ __device__ constexpr size_t simt_px_lds(int tiles_per_wg, int nw, int V) {
  return sizeof(float) * (size_t)tiles_per_wg * nw * V;
}

template <typename T, int M, int R, int CPL, bool NTW, bool PH = false>
__global__ __launch_bounds__(kMaxWaves * kWave) void gemv_simt_px_kernel(
    T* y, const T* x, const T* w, int N, int K, int64_t sxm, int64_t swn, int64_t sym,
    int64_t syn, Epi e, int tiles, int phases) {
  typedef typename Vec8<T>::type V8;
  constexpr int V = pow2_ceil(R * M);
  extern __shared__ __align__(16) float parts[];  // [my tile][wave][V]
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // scalar: the tests below branch once
  const int nt = block_threads(), nw = nt / kWave;
  const int g = (int)gridDim.x;
  const int mine = ((int)blockIdx.x < tiles) ? (tiles - (int)blockIdx.x + g - 1) / g : 0;
  // this lane's CPL K chunks in phase p: chunk p * nw * CPL + wave + c * nw of
  // the row (past K: a dummy address, never used)
  int kc[CPL];
  bool kin[CPL];
  // every chunk of this wave inside K (every wave when the chunks fill the
  // waves evenly): its sums start from the first chunk's products, with no
  // masking and no separate zeroing
  bool whole;
  auto set_phase = [&](int p) {
    const int c0 = p * nw * CPL + wave;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int k = ((c0 + c * nw) * kWave + lane) * 8;
      kin[c] = k < K;
      kc[c] = kin[c] ? k : 0;
    }
    whole = ((c0 + (CPL - 1) * nw) * kWave + kWave - 1) * 8 < K;
  };

  struct Regs {
    V8 v[CPL][R];
  };
  // tile i of this workgroup: its R rows at this lane's chunks (rows past N
  // load the matrix's first 16 bytes, never used)
  auto issue = [&](Regs& q, int i) {
    const int64_t n0 = (int64_t)((int)blockIdx.x + i * g) * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = n0 + r;
      const T* wr = n < N ? w + n * swn : w;  // a wave-uniform row base
#pragma unroll
      for (int c = 0; c < CPL; ++c) q.v[c][r] = load8w<NTW, T>(wr + kc[c]);
    }
  };
  Regs a, b;
  V8 xv[CPL][M];
  bool first = true;  // phase 0: the sums start the LDS slots
  auto consume = [&](const Regs& q, int i) {
    float acc[V];
    if (whole) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r * M + m] = dot8_first(q.v[0][r], xv[0][m]);
#pragma unroll
      for (int c = 1; c < CPL; ++c)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m) acc[r * M + m] = dot8(q.v[c][r], xv[c][m], acc[r * M + m]);
#pragma unroll
      for (int j = R * M; j < V; ++j) acc[j] = 0.f;
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        if (kin[c]) {
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[r * M + m] = dot8(q.v[c][r], xv[c][m], acc[r * M + m]);
        }
      }
    }
    butterfly_sum<V>(acc, lane);
    if (butterfly_writer<V>(lane)) {
      float& slot = parts[(i * nw + wave) * V + butterfly_index<V>(lane)];
      slot = first ? acc[0] : slot + acc[0];
    }
  };
  for (int p = 0; p < (PH ? phases : 1); ++p) {
    set_phase(p);
    if (mine > 0) issue(a, 0);
#pragma unroll
    for (int c = 0; c < CPL; ++c)
#pragma unroll
      for (int m = 0; m < M; ++m) xv[c][m] = load8<T>(x + m * sxm + kc[c]);
    stream_steps(mine, a, b, issue, consume);
    first = false;
  }
  __syncthreads();
  for (int t = tid; t < mine * R * M; t += nt) {
    const int i = t / (R * M), rm = t % (R * M);
    const int r = rm / M, m = rm % M;
    const int64_t n = (int64_t)((int)blockIdx.x + i * g) * R + r;
    if (n < N) {
      float sum = 0.f;
      for (int j = 0; j < nw; ++j) sum += parts[(i * nw + j) * V + rm];
      y[m * sym + n * syn] = from_f32<T>(epilogue(e, sum, m, n));
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA GEMV with row-contiguous weight loads (M padded to 16)
//
// The MFMA A operand wants lane l to hold row l%16, so loading it directly
// makes every load instruction touch 16 rows x 64 bytes: 16 half-used cache
// lines (measured: a pure read in that pattern reaches 5.7 TB/s against 6.9 TB/s
// for row-contiguous 16-byte loads). Here each wave loads its 16 x 128 tile as 4
// instructions of 4 rows x 256 contiguous bytes (lane l: row 4i + l/16, chunk
// l%16), stores it to a wave-private 4 KiB LDS buffer with the 16-byte chunk
// index XOR-swizzled by the row (conflict-free on both sides), and reads it back
// in MFMA layout. Waves split K in 128-element units; with U = 2 each wave keeps
// its next unit's loads in flight while it stages and multiplies the current
// one (stream_steps), with U = 1 one unit at a time.
//
// With ROPE the tile rows follow TileRows<16> and the epilogue rotates the
// rounded outputs of rotated tiles: lanes 0-31 hold slots 0-7 and lanes 32-63
// their partners 8-15 (same m), one lane-xor-32 exchange apart.
// Registers of one 16x128 unit of the MFMA forms: S weight sets (gate/up: 2)
// of four 16-byte row-chunk loads, and the four B (x) fragments.
template <typename T, int S>
struct UnitRegs16 {
  u32x4 v[S][4];
  typename Vec8<T>::type b[4];
};

// Loads of unit u, all unconditional: a lane whose K chunk is past K reads its
// row's first chunk instead (zeroed when staged), a B fragment past K its x
// row's first fragment (zeroed by unit_b). `wl` are weight row bases (rows past
// N clamped by the caller to row 0), `xr` the lane's x row.
template <typename T, int S, bool NTW, bool LOADB = true>
__device__ __forceinline__ void load_unit16(UnitRegs16<T, S>& q, const T* const (&wl)[S][4],
                                            const T* xr, int u, int lchunk, int g, int K) {
  const int k = u * kUnit + lchunk * 8;
  const int kc = k < K ? k : 0;
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4* p = reinterpret_cast<const u32x4*>(wl[s][i] + kc);
      q.v[s][i] = NTW ? __builtin_nontemporal_load(p) : *p;
    }
  if constexpr (LOADB) {
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      const int kb = u * kUnit + (s2 * 4 + g) * 8;
      q.b[s2] = load8<T>(xr + (kb < K ? kb : 0));
    }
  }
}

// Stage a unit's rows (zeros past K) in the wave's LDS tile, row 4i+lrow chunk
// lchunk at slot row*16 + (chunk ^ row), and read back the MFMA A fragments.
template <typename T>
__device__ __forceinline__ void stage_unit16(const u32x4 (&v)[4], u32x4* tile, int lrow,
                                             int lchunk, int u, int K, int r, int g,
                                             typename Vec8<T>::type (&a)[4]) {
  const bool in = u * kUnit + lchunk * 8 < K;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * i + lrow;
    tile[row * 16 + (lchunk ^ row)] = in ? v[i] : u32x4{0, 0, 0, 0};
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2)
    a[s2] = __builtin_bit_cast(typename Vec8<T>::type, tile[r * 16 + ((s2 * 4 + g) ^ r)]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// Generic GEMV: any strides, any K. One workgroup per output column n.

template <typename T>
__global__ __launch_bounds__(256) void gemv_gen_kernel(T* y, const T* x, const T* w, int M,
                                                       int64_t K, int64_t sxm, int64_t sxk,
                                                       int64_t swn, int64_t swk, int64_t sym,
                                                       int64_t syn, Epi e) {
  __shared__ float red[4][16];
  const int64_t n = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  float acc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) acc[m] = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    const float wv = to_f32(w[n * swn + k * swk]);
#pragma unroll
    for (int m = 0; m < 16; ++m)
      if (m < M) acc[m] += wv * to_f32(x[m * sxm + k * sxk]);
  }
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    if (m < M) {
      const float s = wave_sum(acc[m]);
      if (lane == 0) red[wave][m] = s;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < M) {
    const int m = threadIdx.x;
    const float s = red[0][m] + red[1][m] + red[2][m] + red[3][m];
    y[m * sym + n * syn] = from_f32<T>(epilogue(e, s, m, n));
  }
}

// ---------------------------------------------------------------------------
// Fused MLP, launch 1: RMSNorm prologue + gate/up GEMV + SwiGLU epilogue.

// Weight registers of one K step: R gate rows and the matching R up rows.
template <typename T, int R>
struct GateUpRegs {
  typename Vec8<T>::type g[R], u[R];
};

// Loads of step s of the plan. Lanes past H and rows past I load the matrix's
// first 16 bytes instead (never used), so every load is unconditional (see
// stream_steps).
template <typename T, int R, bool NTW>
__device__ __forceinline__ void load_gate_up(GateUpRegs<T, R>& b, const T* wgu,
                                             const StepPlan& p, int s, int H, int I) {
  const int64_t j0 = (int64_t)p.tile(s) * R;
  const int k = p.k(s);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t j = j0 + r;
    const bool ok = j < I && k < H;
    b.g[r] = load8w<NTW, T>(ok ? wgu + j * H + k : wgu);
    b.u[r] = load8w<NTW, T>(ok ? wgu + (I + j) * H + k : wgu);
  }
}

// SIMT gate/up for M < 5 (any M with kind=simt). The weight stream is
// software-pipelined one K step deep over the workgroup's whole sequence of
// (tile, step) pairs: the loads of the next step (which may belong to the next
// tile) are in flight during the math, cross-wave reduction and SwiGLU
// epilogue of the current one, and the first step is issued before the RMSNorm
// prologue's reduction.
template <typename T, int M, int R, bool NTW, bool REGS>
__global__ __launch_bounds__(kMaxWaves * kWave) void mlp_gate_up_simt_kernel(
    T* mid, const T* hidden, const void* nwp, int nw_dtype, const T* wgu, int H, int I,
    float eps, int tiles) {
  typedef typename Vec8<T>::type V8;
  constexpr int V = pow2_ceil(2 * R * M);
  extern __shared__ __align__(16) unsigned char smem[];
  const int XS = xs_stride(H);
  T* xs = reinterpret_cast<T*>(smem);
  float* part = reinterpret_cast<float*>(smem + (size_t)M * XS * sizeof(T));
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = block_threads() / kWave;
  const StepPlan p(tiles, H, nw * kChunk, (wave * kWave + lane) * 8);

  NormRegs<T, M, kNormRegRows(M)> nr;
  if constexpr (REGS) norm_load(nr, hidden, nwp, nw_dtype, M, H);
  GateUpRegs<T, R> a, b;
  load_gate_up<T, R, NTW>(a, wgu, p, 0, H, I);
  if constexpr (REGS)
    norm_store(nr, xs, part, nw_dtype, M, H, eps);
  else
    stage_normed<T, M>(xs, part, hidden, nwp, nw_dtype, M, H, eps);

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  auto issue = [&](GateUpRegs<T, R>& buf, int s) { load_gate_up<T, R, NTW>(buf, wgu, p, s, H, I); };
  auto consume = [&](const GateUpRegs<T, R>& buf, int s) {
    const int k = p.k(s);
    if (k < H) {
      V8 xv[M];
#pragma unroll
      for (int m = 0; m < M; ++m) xv[m] = load8<T>(xs + m * XS + k);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) {
          acc[r * M + m] = dot8(buf.g[r], xv[m], acc[r * M + m]);
          acc[R * M + r * M + m] = dot8(buf.u[r], xv[m], acc[R * M + r * M + m]);
        }
    }
    if (!p.last(s)) return;
    butterfly_sum<V>(acc, lane);
    // Consecutive tiles alternate halves of `part`, so one barrier suffices: the
    // half written here was last read two tiles ago, before the previous barrier.
    float* pt = part + p.half(s) * (V * kMaxWaves);
    if (butterfly_writer<V>(lane)) pt[wave * V + butterfly_index<V>(lane)] = acc[0];
    __syncthreads();
    const int64_t j0 = (int64_t)p.tile(s) * R;
    for (int t = threadIdx.x; t < R * M; t += block_threads()) {
      const int r = t / M, m = t % M;
      const int64_t j = j0 + r;
      if (j < I) {
        float gs = 0.f, us = 0.f;
        for (int i = 0; i < nw; ++i) {
          gs += pt[i * V + t];
          us += pt[i * V + R * M + t];
        }
        mid[m * (int64_t)I + j] = swiglu_out<T>(gs, us);
      }
    }
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
  };
  stream_steps(p.total, a, b, issue, consume);
}

// Pre-attention QKV for M < 5 (and kind=simt): the RMSNorm prologue and step
// pipeline of the fused gate/up kernel over 4 weight rows per tile placed by
// TileRows<4> (two rotate-half pairs per rotated tile), and an epilogue that
// adds the bias, rounds, and rotates the rotated tiles' pairs.
template <typename T, int R>
struct RowRegs {
  typename Vec8<T>::type v[R];
};

template <typename T, int R, bool NTW>
__device__ __forceinline__ void load_tile_rows(RowRegs<T, R>& b, const T* w, const Rope& rp,
                                               const StepPlan& p, int s, int H, int N) {
  const TileRows<R> tr(rp, p.tile(s));
  const int k = p.k(s);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = tr.row(r);
    const bool ok = n < N && k < H;
    b.v[r] = load8w<NTW, T>(ok ? w + n * H + k : w);
  }
}

template <typename T, int M, int R, bool NTW, bool REGS>
__global__ __launch_bounds__(kMaxWaves * kWave) void qkv_simt_kernel(
    T* y, const T* hidden, const void* nwp, int nw_dtype, const T* w, int H, int N, float eps,
    int tiles, Epi e, Rope rp) {
  typedef typename Vec8<T>::type V8;
  constexpr int V = pow2_ceil(R * M);
  extern __shared__ __align__(16) unsigned char smem[];
  const int XS = xs_stride(H);
  T* xs = reinterpret_cast<T*>(smem);
  float* part = reinterpret_cast<float*>(smem + (size_t)M * XS * sizeof(T));
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = block_threads() / kWave;
  const StepPlan p(tiles, H, nw * kChunk, (wave * kWave + lane) * 8);

  NormRegs<T, M, kNormRegRows(M)> nr;
  if constexpr (REGS) norm_load(nr, hidden, nwp, nw_dtype, M, H);
  RowRegs<T, R> a, b;
  load_tile_rows<T, R, NTW>(a, w, rp, p, 0, H, N);
  if constexpr (REGS)
    norm_store(nr, xs, part, nw_dtype, M, H, eps);
  else
    stage_normed<T, M>(xs, part, hidden, nwp, nw_dtype, M, H, eps);

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  auto issue = [&](RowRegs<T, R>& buf, int s) { load_tile_rows<T, R, NTW>(buf, w, rp, p, s, H, N); };
  auto consume = [&](const RowRegs<T, R>& buf, int s) {
    const int k = p.k(s);
    if (k < H) {
      V8 xv[M];
#pragma unroll
      for (int m = 0; m < M; ++m) xv[m] = load8<T>(xs + m * XS + k);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r * M + m] = dot8(buf.v[r], xv[m], acc[r * M + m]);
    }
    if (!p.last(s)) return;
    butterfly_sum<V>(acc, lane);
    // Consecutive tiles alternate halves of `part`, so one barrier suffices: the
    // half written here was last read two tiles ago, before the previous barrier.
    float* pt = part + p.half(s) * (V * kMaxWaves);
    if (butterfly_writer<V>(lane)) pt[wave * V + butterfly_index<V>(lane)] = acc[0];
    __syncthreads();
    qkv_tile_out<T, M, R>(y, pt, V, nw, TileRows<R>(rp, p.tile(s)), e, rp, NoScale{}, N);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
  };
  stream_steps(p.total, a, b, issue, consume);
}

// Fused QKV on the persistent SIMT GEMV (gemv_simt_px_kernel). Every wave loads
// its CPL K chunks of the M hidden rows into registers once; the workgroup adds
// their sums of squares (one barrier) and each wave normalises its chunks in
// place, round(x * inv * w) as stage_normed does. The tiles of R weight rows,
// placed by TileRows<R> (R/2 rotate-half pairs of one head, or R consecutive
// rows past rope_cols), then stream as in the GEMV with the normalised rows
// in registers, and after the last tile the workgroup adds the waves' sums,
// applies the bias, rounds, and rotates the pairs of rotated tiles.
template <typename T, int M, int R, int CPL, bool NTW>
__global__ __launch_bounds__(kMaxWaves * kWave) void qkv_px_kernel(
    T* y, const T* x, const void* nwp, int nw_dtype, const T* w, int H, int N, float eps,
    int tiles, Epi e, Rope rp) {
  typedef typename Vec8<T>::type V8;
  constexpr int V = pow2_ceil(R * M);
  constexpr int MP = pow2_ceil(M);
  constexpr int P = R / 2;
  extern __shared__ __align__(16) float pxs[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int nt = block_threads(), nw = nt / kWave;
  const int g = (int)gridDim.x;
  const int mine = ((int)blockIdx.x < tiles) ? (tiles - (int)blockIdx.x + g - 1) / g : 0;
  float* parts = pxs;                                 // [my tile][wave][V]
  float* ssq = pxs + (size_t)mine * nw * V;           // [wave][MP]
  float* inv = ssq + kMaxWaves * MP;                  // [MP]
  int kc[CPL];
  bool kin[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int k = ((wave + c * nw) * kWave + lane) * 8;
    kin[c] = k < H;
    kc[c] = kin[c] ? k : 0;
  }
  const bool whole = ((wave + (CPL - 1) * nw) * kWave + kWave - 1) * 8 < H;

  struct Regs {
    V8 v[CPL][R];
  };
  auto issue = [&](Regs& q, int i) {
    const TileRows<R> tr(rp, (int)blockIdx.x + i * g);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = tr.row(r);
      const T* wr = n < N ? w + n * H : w;  // a wave-uniform row base
#pragma unroll
      for (int c = 0; c < CPL; ++c) q.v[c][r] = load8w<NTW, T>(wr + kc[c]);
    }
  };
  // the rows and the norm weight first, then the first tile's weights: the norm
  // waits only for its own loads (they complete in issue order) while the tile
  // streams (Llama-3-8B QKV, M = 5 / 8: 12.4 / 13.7 us, against 13.3 / 13.9
  // with the tile issued first and 12.7 / 14.4 with two tiles issued here)
  V8 xv[CPL][M];
  float wf[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
#pragma unroll
    for (int m = 0; m < M; ++m) xv[c][m] = load8<T>(x + (int64_t)m * H + kc[c]);
    load8_norm_w(nwp, nw_dtype, kc[c], wf[c]);
  }
  Regs a, b;
  if (mine > 0) issue(a, 0);
  // RMSNorm: the rows' sums of squares over this lane's chunks (v_dot2 of each
  // pair with itself), the waves', then the workgroup's; every wave normalises
  // its own chunks (norm_frag: x * inv as one v_fma_mix for fp16)
  float ss[MP];
#pragma unroll
  for (int m = 0; m < MP; ++m) ss[m] = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c)
    if (kin[c]) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const u32x4 u = __builtin_bit_cast(u32x4, xv[c][m]);
#pragma unroll
        for (int j = 0; j < 4; ++j) ss[m] = sq_dot2<T>(u[j], ss[m]);
      }
    }
  butterfly_sum<MP>(ss, lane);
  if (butterfly_writer<MP>(lane)) ssq[wave * MP + butterfly_index<MP>(lane)] = ss[0];
  __syncthreads();
  if (tid < M) {
    float s = 0.f;
    for (int i = 0; i < nw; ++i) s += ssq[i * MP + tid];
    inv[tid] = rsqrtf(s / (float)H + eps);
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const u32x4 w0 = __builtin_bit_cast(u32x4, f32x4{wf[c][0], wf[c][1], wf[c][2], wf[c][3]});
    const u32x4 w1 = __builtin_bit_cast(u32x4, f32x4{wf[c][4], wf[c][5], wf[c][6], wf[c][7]});
#pragma unroll
    for (int m = 0; m < M; ++m)
      xv[c][m] = __builtin_bit_cast(V8, norm_frag<T>(__builtin_bit_cast(u32x4, xv[c][m]), inv[m], w0, w1));
  }
  auto consume = [&](const Regs& q, int i) {
    float acc[V];
    if (whole) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r * M + m] = dot8_first(q.v[0][r], xv[0][m]);
#pragma unroll
      for (int c = 1; c < CPL; ++c)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m) acc[r * M + m] = dot8(q.v[c][r], xv[c][m], acc[r * M + m]);
#pragma unroll
      for (int j = R * M; j < V; ++j) acc[j] = 0.f;
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        if (kin[c]) {
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[r * M + m] = dot8(q.v[c][r], xv[c][m], acc[r * M + m]);
        }
      }
    }
    butterfly_sum<V>(acc, lane);
    if (butterfly_writer<V>(lane)) parts[(i * nw + wave) * V + butterfly_index<V>(lane)] = acc[0];
  };
  stream_steps(mine, a, b, issue, consume);
  __syncthreads();
  for (int t = tid; t < mine * R * M; t += nt) {
    const int i = t / (R * M), rm = t % (R * M);
    const TileRows<R> tr(rp, (int)blockIdx.x + i * g);
    const float* pt = parts + (size_t)i * nw * V;
    if (tr.rotated()) {
      if (rm >= P * M) continue;  // one item per rotate-half pair
      const int p = rm / M, m = rm % M;
      float s1 = 0.f, s2 = 0.f;
      for (int j = 0; j < nw; ++j) {
        s1 += pt[j * V + p * M + m];
        s2 += pt[j * V + (p + P) * M + m];
      }
      const int64_t n1 = tr.row(p), n2 = tr.row(p + P);
      float o1, o2;
      rope_pair(rp, m, tr.col(p), round_as<T>(epilogue(e, s1, m, n1)), round_as<T>(epilogue(e, s2, m, n2)), o1,
                o2);
      y[m * (int64_t)N + n1] = from_f32<T>(o1);
      y[m * (int64_t)N + n2] = from_f32<T>(o2);
    } else {
      const int r = rm / M, m = rm % M;
      const int64_t n = tr.row(r);
      if (n < N) {
        float s = 0.f;
        for (int j = 0; j < nw; ++j) s += pt[j * V + rm];
        y[m * (int64_t)N + n] = from_f32<T>(epilogue(e, s, m, n));
      }
    }
  }
}

// MFMA form of the gate/up launch for M >= kMfmaMinM (M padded to 16): a tile of
// 16 gate rows and the matching 16 up rows per workgroup, streamed with the
// row-contiguous load + LDS relayout of gemv_mfma_relayout_kernel. B operand:
// the activations from global memory (L2-resident, [M, H]). Without SS they
// are the normalised rows a separate row kernel wrote (into the caller's output
// buffer, which the down projection overwrites last; from 9 rows).
//
// With SS, x is the raw hidden state and the kernel normalises it itself from
// the row sums of squares its producer wrote (RowSq): the prologue stages the
// norm weight as float32 in LDS and derives inv[m] from those sums, and every B
// fragment becomes round(x * inv[m] * w[k]) before its MFMA -- the row kernel's
// arithmetic, without its launch. Launched with at most kSsWaves waves, and
// held to the VGPRs of three waves per SIMD (the form without SS needs as
// many).

//
// HALF (M <= 8): the activation fragments in the half-B form (load_b_half).
// FX (with SS): no producer sums; the prologue derives the row sums from x
// (up to 8 rows: every workgroup reads the rows from L2 once more, which costs
// less than the row kernel's launch).
//
// SPLIT: a tile of 8 gate rows (from j0) and their 8 up rows, one 16-row weight
// set per unit (one relayout, four MFMAs); output rows 0-7 (gate) sit in lanes
// 0-31 and their up rows 8-15 in lanes 32-63, so the epilogue pairs lane t
// with t + 32. Each activation fragment then feeds half the MFMAs, so these
// tiles only take the rows past the last whole round of 16 + 16 tiles over the
// CUs (relayout_grid).
template <typename T, bool NTW, bool SS, bool HALF, bool FX, bool SPLIT>
__device__ __forceinline__ void gate_up_relayout_tile(f32x4* part, u32x4 (*tiles)[256], int64_t j0, T* mid,
                                                      const T* x, const T* wgu, int M, int H, int I,
                                                      const void* nwp, int nw_dtype, float eps, const RowSq& rq) {
  typedef typename Vec8<T>::type V8;
  constexpr int S = SPLIT ? 1 : 2;  // weight sets per unit
  extern __shared__ float norm_lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = block_threads() / kWave;
  const int r = lane & 15, g = lane >> 4;
  const int hi = r >= 8, xrow = HALF ? half_b_row(r) : r;
  const T* xr = x + (xrow < M ? xrow : 0) * (int64_t)H;  // rows past M: columns never stored
  const int lrow = lane >> 4, lchunk = lane & 15;
  const T* wl[S][4];  // [gate, up][row 4i + lrow] bases; SPLIT: tile row 4i + lrow
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (SPLIT) {
      const int64_t j = j0 + ((4 * i + lrow) & 7);
      const int64_t jc = j < I ? j : 0;
      wl[0][i] = wgu + (i < 2 ? jc : I + jc) * H;  // rows 0-7 gate, 8-15 up
    } else {
      const int64_t j = j0 + 4 * i + lrow;
      const int64_t jc = j < I ? j : 0;
      wl[0][i] = wgu + jc * H;
      wl[S - 1][i] = wgu + (I + jc) * H;
    }
  }
  u32x4* tile = tiles[wave];
  f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
  const int units = (H + kUnit - 1) / kUnit;
  const int mine = wave < units ? (units - wave + nw - 1) / nw : 0;
  const int off = sweep_offset(units);
  auto issue = [&](UnitRegs16<T, S>& q, int i) {
    const int u = sweep_unit(wave, i, nw, off, units);
    load_unit16<T, S, NTW, !HALF>(q, wl, xr, u, lchunk, g, H);
    if constexpr (HALF) load_b_half<T>(q.b, xr, u, g, hi, H);
  };
  float rinv = 0.f;
  // fragment s2's B: the activations, normalised in the SS form, zero past K
  auto frag = [&](const V8& raw, int u, int s2) {
    V8 xb = raw;
    if constexpr (SS) {
      const f32x4* wk = reinterpret_cast<const f32x4*>(norm_lds + u * kUnit + (s2 * 4 + g) * 8);
      xb = __builtin_bit_cast(V8, norm_frag<T>(__builtin_bit_cast(u32x4, xb), rinv,
                                               __builtin_bit_cast(u32x4, wk[0]),
                                               __builtin_bit_cast(u32x4, wk[1])));
    }
    return unit_b(xb, u, s2, g, H);
  };
  auto consume = [&](const UnitRegs16<T, S>& q, int i) {
    const int u = sweep_unit(wave, i, nw, off, units);
    V8 a[4], c[4];
    stage_unit16<T>(q.v[0], tile, lrow, lchunk, u, H, r, g, a);
    if constexpr (!SPLIT) stage_unit16<T>(q.v[S - 1], tile, lrow, lchunk, u, H, r, g, c);
    if constexpr (HALF) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const V8 own = frag(q.b[p], u, 2 * p + hi);
        const V8 oth = __builtin_bit_cast(V8, mirror16(__builtin_bit_cast(u32x4, own)));
        ag = mfma16(a[2 * p], own, ag);
        if constexpr (!SPLIT) au = mfma16(c[2 * p], own, au);
        ag = mfma16(a[2 * p + 1], oth, ag);
        if constexpr (!SPLIT) au = mfma16(c[2 * p + 1], oth, au);
      }
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        const V8 b = frag(q.b[s2], u, s2);
        ag = mfma16(a[s2], b, ag);
        if constexpr (!SPLIT) au = mfma16(c[s2], b, au);
      }
    }
  };
  UnitRegs16<T, S> qa, qb;
  if constexpr (SS) {  // the first unit's loads fly while the prologue runs
    float* inv = norm_lds + units * kUnit;
    norm_prologue<T, HALF ? 8 : 16, FX, kSsWaves * kWave>(norm_lds, inv, inv + 16, nwp, nw_dtype, x, H, M, H,
                                                         units * kUnit, eps, rq, [&] {
                                                           if (mine > 0) issue(qa, 0);
                                                         });
    rinv = inv[xrow];
  } else {
    if (mine > 0) issue(qa, 0);
  }
  stream_steps(mine, qa, qb, issue, consume);
  if constexpr (SPLIT) {  // one reduction: lane t < 32 adds the gate sums of t, the up sums of t + 32
    part[wave * kWave + lane] = ag;
    __syncthreads();
    if (threadIdx.x < 32) {
      f32x4 sg = part[threadIdx.x], su = part[threadIdx.x + 32];
      for (int i = 1; i < nw; ++i) {
        sg += part[i * kWave + threadIdx.x];
        su += part[i * kWave + threadIdx.x + 32];
      }
      const int m = threadIdx.x & 15;
      const int nb = (threadIdx.x >> 4) * 4;
      if (m < M) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t jj = j0 + nb + i;
          if (jj < I) mid[m * (int64_t)I + jj] = swiglu_out<T>(sg[i], su[i]);
        }
      }
    }
    return;
  }
  // two-phase reduction through one buffer: gate sums, then up sums
  part[wave * kWave + lane] = ag;
  __syncthreads();
  f32x4 sg = {0.f, 0.f, 0.f, 0.f};
  if (threadIdx.x < kWave)
    for (int i = 0; i < nw; ++i) sg += part[i * kWave + threadIdx.x];
  __syncthreads();
  part[wave * kWave + lane] = au;
  __syncthreads();
  if (threadIdx.x < kWave) {
    f32x4 su = part[threadIdx.x];
    for (int i = 1; i < nw; ++i) su += part[i * kWave + threadIdx.x];
    const int m = threadIdx.x & 15;
    const int nb = (threadIdx.x >> 4) * 4;
    if (m < M) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t jj = j0 + nb + i;
        if (jj < I) mid[m * (int64_t)I + jj] = swiglu_out<T>(sg[i], su[i]);
      }
    }
  }
}

// The gate/up launch: workgroup b < big takes 16 gate + 16 up rows from 16 b;
// with MIX the rest take 8 + 8 rows each after those (relayout_grid).
template <typename T, bool NTW, bool SS, bool HALF, bool FX = false, bool MIX = false>
__global__ __launch_bounds__(SS || HALF ? kSsWaves * kWave : kMaxWaves * kWave, SS || HALF ? 3 : 1) void mlp_gate_up_relayout_kernel(
    T* mid, const T* x, const T* wgu, int M, int H, int I, const void* nwp, int nw_dtype, float eps,
    RowSq rq, int big) {
  constexpr int LW = SS ? kSsWaves : kMaxWaves;
  __shared__ f32x4 part[LW * kWave];
  __shared__ u32x4 tiles[LW][256];
  const int b = (int)blockIdx.x;
  if constexpr (MIX) {
    if (b >= big) {
      gate_up_relayout_tile<T, NTW, SS, HALF, FX, true>(part, tiles, (int64_t)big * 16 + (int64_t)(b - big) * 8, mid,
                                                        x, wgu, M, H, I, nwp, nw_dtype, eps, rq);
      return;
    }
  }
  gate_up_relayout_tile<T, NTW, SS, HALF, FX, false>(part, tiles, (int64_t)b * 16, mid, x, wgu, M, H, I, nwp,
                                                     nw_dtype, eps, rq);
}

// ---------------------------------------------------------------------------
// Host side

namespace {

// kind=dot runs the MFMA GEMV from this M on unless a tile names the other kernel:
// the tile table does so per shape where the tile search measured it faster
// (MFMA already at M = 3-4 on N = 28672 and K = 14336, the persistent SIMT kernel
// still at M = 5-9 on N = 6144). The fused MLP and QKV take their MFMA routes, and the row-sum
// handoff runs, from this M on.
constexpr int kMfmaMinM = 5;

// Tiling of one GEMV launch; 0 = the default for the kernel that runs.
struct Tile {
  int rows;    // weight rows per workgroup (SIMT 2, 4, 8; MFMA 16)
  int waves;   // waves per workgroup, 1..8
  int stages;  // MFMA: K units in flight per wave (1-3); SIMT: 1 per-tile, 2 persistent kernel
};

template <typename T, int M, int R>
void launch_simt_r(void* y, const void* x, const void* w, int N, int K, int64_t sxm, int64_t swn,
                   int64_t sym, int64_t syn, const Epi& e, int nw, hipStream_t st) {
  const unsigned blocks = (unsigned)((N + R - 1) / R);
  hipLaunchKernelGGL((gemv_simt_kernel<T, M, R, kNtWeights>), dim3(blocks), dim3(nw * kWave), 0, st,
                     static_cast<T*>(y), static_cast<const T*>(x), static_cast<const T*>(w), N,
                     K, sxm, swn, sym, syn, e);
}

// The persistent SIMT GEMV: `cpl` 512-element K chunks per lane (1, 2 or 4),
// ceil(chunks / cpl) waves of at most eight, a grid of one or two workgroups
// per CU (simt_px_grid; fewer when the tiles are fewer), each owning every
// gridDim-th tile; LDS holds its tiles' per-wave sums.
inline int simt_px_waves(int K, int cpl) {
  const int chunks = (K + kChunk - 1) / kChunk;
  return (chunks + cpl - 1) / cpl;
}

// Phases of the persistent SIMT GEMV: the fewest runs of at most eight waves x
// cpl chunks that cover K, and the waves that spread the chunks evenly over
// them (K = 14336, cpl = 2: two phases of seven waves).
struct PxPhases {
  int phases, waves;
};
inline PxPhases simt_px_phases(int K, int cpl) {
  const int chunks = (K + kChunk - 1) / kChunk;
  const int ph = (chunks + kMaxWaves * cpl - 1) / (kMaxWaves * cpl);
  return {ph, (chunks + ph * cpl - 1) / (ph * cpl)};
}

// Workgroups of the persistent SIMT GEMV. Each one reads all M activation rows
// into registers (M*K elements from L2) before its first tile, so a second
// workgroup per CU pays off only while the weight rows each one streams still
// outweigh that: two per CU where N >= 4*M*CUs, else one (M = 8, K = 4096:
// N = 4096 9.05 -> 8.67 us and N = 6144 11.86 -> 11.78 with one per CU,
// N = 4096 K = 14336 26.2 -> 24.9, but N = 28672 40.9 -> 42.9).
inline bool simt_px_one_per_cu(int N, int M) { return N < 4 * M * device_cus(); }
inline int simt_px_grid(int N, int M, int tiles) {
  const int grid = (simt_px_one_per_cu(N, M) ? 1 : 2) * device_cus();
  return grid < tiles ? grid : tiles;
}

template <typename T, int M, int R, int CPL>
int launch_simt_px_r(void* y, const void* x, const void* w, int N, int K, int64_t sxm, int64_t swn,
                     int64_t sym, int64_t syn, const Epi& e, hipStream_t st) {
  constexpr int V = pow2_ceil(R * M);
  if (K <= 0) return set_error(FD_EUNSUPPORTED, "the persistent SIMT GEMV needs K > 0");
  const PxPhases ph = simt_px_phases(K, CPL);
  const int nw = ph.waves;
  const int tiles = (N + R - 1) / R;
  const int grid = simt_px_grid(N, M, tiles);
  const int per = (tiles + grid - 1) / grid;
  const size_t lds = simt_px_lds(per, nw, V);
  if (lds > kMaxLds / 2) return set_error(FD_EUNSUPPORTED, "too many tiles per workgroup for the LDS sums");
  auto kernel = ph.phases > 1 ? gemv_simt_px_kernel<T, M, R, CPL, kNtWeights, true>
                              : gemv_simt_px_kernel<T, M, R, CPL, kNtWeights, false>;
  if (!allow_lds(kernel, lds)) return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", lds);
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(nw * kWave), lds, st, static_cast<T*>(y),
                     static_cast<const T*>(x), static_cast<const T*>(w), N, K, sxm, swn, sym, syn, e, tiles,
                     ph.phases);
  return FD_OK;
}

// K chunks per lane of the persistent SIMT GEMV: what `waves` asks for (the
// chunks spread over that many waves, rounded up to 1, 2 or 4), else the
// fewest that keep K within eight waves, and two from 5 rows: the butterfly per
// tile then covers twice the products (K = 4096, M = 8: N = 4096 9.30 against
// 9.92 us, N = 28672 39.47 against 42.09; M = 16: 12.30 against 12.93, 55.89
// against 65.96).
inline int simt_px_cpl(int M, int K, int waves) {
  const int chunks = (K + kChunk - 1) / kChunk;
  int cpl = waves > 0 ? (chunks + waves - 1) / waves : (chunks + kMaxWaves - 1) / kMaxWaves;
  if (waves <= 0 && M >= 5 && cpl < 2) cpl = 2;
  return cpl <= 1 ? 1 : cpl <= 2 ? 2 : 4;
}

// Register budget of the persistent SIMT GEMV (VGPRs per lane): the CPL*M
// activation vectors, two buffers of R*CPL weight vectors and the padded sums,
// at most 224 (beyond that the compiler spills: M = 16, 4 rows, 2 chunks).
__host__ __device__ constexpr bool simt_px_regs_ok(int M, int R, int cpl) {
  return cpl * M * 4 + 8 * R * cpl + pow2_ceil(R * M) <= 224;
}

// Can the persistent SIMT GEMV take this launch (R rows per tile, cpl chunks
// per lane; in one phase unless `phased`)?
inline bool simt_px_fits(int N, int K, int R, int M, int cpl, bool phased = false) {
  if (K <= 0 || !simt_px_regs_ok(M, R, cpl)) return false;
  const PxPhases ph = simt_px_phases(K, cpl);
  if (ph.phases > 1 && !phased) return false;
  const int tiles = (N + R - 1) / R;
  const int grid = simt_px_grid(N, M, tiles);
  const int per = (tiles + grid - 1) / grid;
  return simt_px_lds(per, ph.waves, pow2_ceil(R * M)) <= kMaxLds / 2;
}

// Default rows per tile of the persistent SIMT GEMV: up to 4 rows, 4; with
// more than one K chunk per lane, 4 where one workgroup per CU runs and the
// registers hold them (M = 8, K = 4096, one per CU: N = 4096 8.67 -> 8.54 us,
// N = 6144 11.78 -> 11.29), else 2.
template <int M>
inline int simt_px_rows(int N, int cpl) {
  if (cpl <= 1) return SimtPxRows<M>::R;
  return M <= 8 && simt_px_one_per_cu(N, M) && simt_px_regs_ok(M, 4, cpl) ? 4 : 2;
}

template <typename T, int M, int R>
int launch_simt_px_c(int cpl, void* y, const void* x, const void* w, int N, int K, int64_t sxm, int64_t swn,
                     int64_t sym, int64_t syn, const Epi& e, hipStream_t st) {
  if (cpl == 1) return launch_simt_px_r<T, M, R, 1>(y, x, w, N, K, sxm, swn, sym, syn, e, st);
  if constexpr (simt_px_regs_ok(M, R, 2))
    if (cpl == 2) return launch_simt_px_r<T, M, R, 2>(y, x, w, N, K, sxm, swn, sym, syn, e, st);
  if constexpr (simt_px_regs_ok(M, R, 4))
    if (cpl == 4) return launch_simt_px_r<T, M, R, 4>(y, x, w, N, K, sxm, swn, sym, syn, e, st);
  return set_error(FD_EUNSUPPORTED, "the persistent SIMT GEMV's registers do not hold M = %d with %d rows and "
                   "%d chunks per lane", M, R, cpl);
}

// Default: 4 rows, waves = one per 512-element K chunk up to 8; from 2 rows the
// persistent kernel where its registers hold the rows (stages 0 or 2; with
// stages 2 the tile's waves set the chunks per lane), in phases where K is past
// eight waves of those chunks, else (or with stages 1) the per-tile kernel. Rows
// 8 exist up to M = 8 (R*M accumulators per lane).
template <typename T, int M>
int launch_simt(void* y, const void* x, const void* w, int N, int K, int64_t sxm, int64_t swn,
                int64_t sym, int64_t syn, const Epi& e, const Tile& t, hipStream_t st) {
  const int nw = t.waves ? t.waves : pick_waves((K + kChunk - 1) / kChunk);
  // (K = 0 has no chunk: the per-tile kernel writes the bias/row_add-only outputs)
  const bool waves_set = t.stages == 2 && t.waves > 0;
  int cpl = simt_px_cpl(M, K, waves_set ? t.waves : 0);
  const int px_rows = t.rows ? t.rows : simt_px_rows<M>(N, cpl);
  // defaulted chunks per lane step down until the registers hold them; K past
  // eight waves of them runs in phases (9-16 rows at K = 14336: two phases of
  // seven waves x two chunks, which read the activations once per phase per
  // workgroup where the per-tile kernel reads them once per tile)
  while (!waves_set && cpl > 1 && !simt_px_regs_ok(M, px_rows, cpl)) cpl /= 2;
  const bool px = t.stages == 2 || (t.stages == 0 && M >= 2 && simt_px_fits(N, K, px_rows, M, cpl, true));
  const int rows = t.rows ? t.rows : px ? px_rows : SimtRows<M>::R;
  const int r = rows == 2 ? 2 : rows == 8 && M <= 8 ? 8 : 4;
  constexpr int R8 = M <= 8 ? 8 : 4;
  if (px) {
    if (r == 2) return launch_simt_px_c<T, M, 2>(cpl, y, x, w, N, K, sxm, swn, sym, syn, e, st);
    if (r == 8) return launch_simt_px_c<T, M, R8>(cpl, y, x, w, N, K, sxm, swn, sym, syn, e, st);
    return launch_simt_px_c<T, M, 4>(cpl, y, x, w, N, K, sxm, swn, sym, syn, e, st);
  }
  if (r == 2)
    launch_simt_r<T, M, 2>(y, x, w, N, K, sxm, swn, sym, syn, e, nw, st);
  else if (r == 8)
    launch_simt_r<T, M, R8>(y, x, w, N, K, sxm, swn, sym, syn, e, nw, st);
  else
    launch_simt_r<T, M, 4>(y, x, w, N, K, sxm, swn, sym, syn, e, nw, st);
  return FD_OK;
}

template <typename T>
int launch_simt_m(int M, void* y, const void* x, const void* w, int N, int K, int64_t sxm,
                  int64_t swn, int64_t sym, int64_t syn, const Epi& e, const Tile& t,
                  hipStream_t st) {
  switch (M) {
#define FD_CASE(MM) \
  case MM: return launch_simt<T, MM>(y, x, w, N, K, sxm, swn, sym, syn, e, t, st);
    FD_CASE(1) FD_CASE(2) FD_CASE(3) FD_CASE(4) FD_CASE(5) FD_CASE(6) FD_CASE(7) FD_CASE(8)
    FD_CASE(9) FD_CASE(10) FD_CASE(11) FD_CASE(12) FD_CASE(13) FD_CASE(14) FD_CASE(15)
    FD_CASE(16)
#undef FD_CASE
    default: return set_error(FD_EINVAL, "M must be in [1, 16]");
  }
}

// Shapes of the DMA MFMA GEMV a tile may name: waves 2, 4 or 8, units in flight
// 1-3, within the LDS of one CU.
inline bool dma_shape_ok(int nw, int d, int M) {
  return (nw == 2 || nw == 4 || nw == 8) && d >= 1 && d <= 3 && dma_lds(nw, d, dma_rows(M)) <= kMaxLds;
}

// Default shape: four waves (fewer when K has fewer units) with two units in
// flight each; measured best or within 3% of the best of 2-8 waves and 1-3
// units on the four decode shapes at M = 5, 8 and 16 (e.g. N = K = 4096, M = 8:
// 7.2 us, against 8.6 for the relayout kernel this replaced, whose two units per
// wave sat in 114 VGPRs). The fused QKV (rp) always runs the default shape.
template <typename T>
int launch_mfma(int M, void* y, const void* x, const void* w, int N, int K, int64_t sxm,
                int64_t swn, int64_t sym, int64_t syn, const Epi& e, hipStream_t st,
                const Rope* rp = nullptr, const Tile* t = nullptr, const FoldNorm* fold = nullptr) {
  const int units = (K + kUnit - 1) / kUnit;
  const int nw = t && t->waves ? t->waves : units >= 4 ? 4 : units >= 2 ? 2 : 1;
  const int d = t && t->stages ? t->stages : 2;
  Rope none{};
  const FoldNorm nofold{nullptr, FD_F32, 0.f};
  const unsigned blocks =
      rp ? (unsigned)(rp->tiles + (N - rp->cols + 15) / 16) : (unsigned)((N + 15) / 16);
  const Rope& r = rp ? *rp : none;
  if (fold)  // the fused QKV from kMfmaMinM rows: RoPE epilogue, RMSNorm folded in
    return launch_dma_default<T, T, EPI_ROPE, true>(blocks, y, x, w, nullptr, M, N, K, sxm, swn, sym, syn, e,
                                                    r, *fold, st);
  if (rp)
    return launch_dma_default<T, T, EPI_ROPE, false>(blocks, y, x, w, nullptr, M, N, K, sxm, swn, sym, syn,
                                                     e, r, nofold, st);
#define FD_DMA(NW, D)                                                                                        \
  return launch_dma_rows<T, T, NW, D, EPI_PLAIN, false>(blocks, y, x, w, nullptr, M, N, K, sxm, swn, sym, syn, \
                                                        e, r, nofold, st)
  if (nw <= 2) {
    if (d == 1) FD_DMA(2, 1); else if (d == 2) FD_DMA(2, 2); else FD_DMA(2, 3);
  } else if (nw <= 4) {
    if (d == 1) FD_DMA(4, 1); else if (d == 2) FD_DMA(4, 2); else FD_DMA(4, 3);
  } else {
    if (d == 1) FD_DMA(8, 1); else if (d == 2) FD_DMA(8, 2); else FD_DMA(8, 3);
  }
#undef FD_DMA
}

template <typename T, int M>
int launch_mlp_simt(void* mid, const void* hidden, const void* nw, int nw_dtype, const void* wgu,
                    int H, int I, float eps, hipStream_t st) {
  constexpr int R = MlpRows<M>::R;
  constexpr int V = pow2_ceil(2 * R * M);
  // Up to 4 rows: eight waves (one 512-element K chunk per row each at
  // H=4096) in one workgroup per CU (Llama-3-8B widths, M=1..4: 34.9 / 35.3 /
  // 36.9 / 37.4 us against 35.7 / 36.1 for two 8-wave workgroups per CU at
  // M=1..2 and 38.5 / 39.2 for two 4-wave ones at M=3..4). Above, where 2*R*M
  // sums per lane cost VGPRs, four waves. Workgroups per CU keep about eight
  // waves per CU resident.
  const int nwv0 = pick_waves((H + kChunk - 1) / kChunk);
  const int nwv = M > 4 && nwv0 > 4 ? 4 : nwv0;
  const size_t lds = fused_lds(M, H, sizeof(T), V);
  if (lds > kMaxLds) return set_error(FD_EUNSUPPORTED, "M*H too large for the LDS stage");
  const int tiles = (I + R - 1) / R;
  const int grid = fused_grid(tiles, lds, kMaxWaves / nwv);
  auto launch = [&](auto kernel) {
    if (!allow_lds(kernel, lds))
      return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", lds);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(nwv * kWave), lds, st, static_cast<T*>(mid),
                       static_cast<const T*>(hidden), nw, nw_dtype, static_cast<const T*>(wgu), H,
                       I, eps, tiles);
    return (int)FD_OK;
  };
  if constexpr (M <= kNormRegMaxM) {
    if (norm_in_regs(M, H, nwv * kWave))
      return launch(mlp_gate_up_simt_kernel<T, M, R, kNtWeights, true>);
  }
  return launch(mlp_gate_up_simt_kernel<T, M, R, kNtWeights, false>);
}

template <typename T>
int launch_mlp_simt_m(int M, void* mid, const void* hidden, const void* nw, int nw_dtype,
                      const void* wgu, int H, int I, float eps, hipStream_t st) {
  switch (M) {
#define FD_CASE(MM) \
  case MM: return launch_mlp_simt<T, MM>(mid, hidden, nw, nw_dtype, wgu, H, I, eps, st);
    FD_CASE(1) FD_CASE(2) FD_CASE(3) FD_CASE(4) FD_CASE(5) FD_CASE(6) FD_CASE(7) FD_CASE(8)
    FD_CASE(9) FD_CASE(10) FD_CASE(11) FD_CASE(12) FD_CASE(13) FD_CASE(14) FD_CASE(15)
    FD_CASE(16)
#undef FD_CASE
    default: return set_error(FD_EINVAL, "M must be in [1, 16]");
  }
}

template <typename T, int M>
int launch_qkv_simt(void* y, const void* hidden, const void* nw, int nw_dtype, const void* w,
                    int H, int N, float eps, const Epi& e, const Rope& rp_in, hipStream_t st) {
  constexpr int R = QkvRows<M>::R;
  constexpr int V = pow2_ceil(R * M);
  // Four waves and every tile resident at once (one tile per workgroup at
  // N = 6144): the QKV weights are too few to amortise a persistent loop.
  const int nwv0 = pick_waves((H + kChunk - 1) / kChunk);
  const int nwv = nwv0 > 4 ? 4 : nwv0;
  const size_t lds = fused_lds(M, H, sizeof(T), V);
  if (lds > kMaxLds) return set_error(FD_EUNSUPPORTED, "M*H too large for the LDS stage");
  Rope rp = rp_in;
  rp.tiles = rp.cols / R;
  const int tiles = rp.tiles + (N - rp.cols + R - 1) / R;
  const int grid = fused_grid(tiles, lds, 8);
  auto launch = [&](auto kernel) {
    if (!allow_lds(kernel, lds))
      return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", lds);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(nwv * kWave), lds, st, static_cast<T*>(y),
                       static_cast<const T*>(hidden), nw, nw_dtype, static_cast<const T*>(w), H, N,
                       eps, tiles, e, rp);
    return (int)FD_OK;
  };
  if constexpr (M <= kNormRegMaxM) {
    if (norm_in_regs(M, H, nwv * kWave)) return launch(qkv_simt_kernel<T, M, R, kNtWeights, true>);
  }
  return launch(qkv_simt_kernel<T, M, R, kNtWeights, false>);
}

// The persistent SIMT form of the fused QKV: the GEMV's launch shape (K chunks
// per lane from simt_px_cpl, workgroups from simt_px_grid, rows per tile from
// simt_px_rows, all even so rotated tiles hold whole pairs). Its LDS holds the
// tiles' per-wave sums and the norm's per-wave sums of squares.
template <typename T, int M, int R, int CPL>
int launch_qkv_px_r(void* y, const void* hidden, const void* nw, int nw_dtype, const void* w, int H, int N,
                    float eps, const Epi& e, Rope rp, hipStream_t st) {
  constexpr int V = pow2_ceil(R * M), MP = pow2_ceil(M);
  const int nwv = simt_px_waves(H, CPL);
  rp.tiles = rp.cols / R;
  const int tiles = rp.tiles + (N - rp.cols + R - 1) / R;
  const int grid = simt_px_grid(N, M, tiles);
  const int per = (tiles + grid - 1) / grid;
  const size_t lds = sizeof(float) * ((size_t)per * nwv * V + kMaxWaves * MP + MP);
  auto kernel = qkv_px_kernel<T, M, R, CPL, kNtWeights>;
  if (!allow_lds(kernel, lds)) return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", lds);
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(nwv * kWave), lds, st, static_cast<T*>(y),
                     static_cast<const T*>(hidden), nw, nw_dtype, static_cast<const T*>(w), H, N, eps, tiles, e, rp);
  return FD_OK;
}

// Chunks per lane and rows per tile of the persistent SIMT QKV, as the GEMV
// would choose them for [N, H] weights; false where that kernel cannot take H
// (more than 8 waves of 4 chunks) or its LDS sums.
template <int M>
bool qkv_px_shape(int N, int H, int& rows, int& cpl) {
  cpl = simt_px_cpl(M, H, 0);
  rows = simt_px_rows<M>(N, cpl);
  while (cpl > 1 && !simt_px_regs_ok(M, rows, cpl) && simt_px_waves(H, cpl / 2) <= kMaxWaves) cpl /= 2;
  return simt_px_fits(N, H, rows, M, cpl);
}

template <typename T, int M>
int launch_qkv_px(void* y, const void* hidden, const void* nw, int nw_dtype, const void* w, int H, int N,
                  float eps, const Epi& e, const Rope& rp, hipStream_t st) {
  int rows = 0, cpl = 0;
  if (!qkv_px_shape<M>(N, H, rows, cpl))
    return set_error(FD_EUNSUPPORTED, "the persistent SIMT QKV does not take H = %d", H);
  auto go = [&](auto rtag, auto ctag) -> int {
    constexpr int RR = decltype(rtag)::value, CC = decltype(ctag)::value;
    if constexpr (simt_px_regs_ok(M, RR, CC))
      return launch_qkv_px_r<T, M, RR, CC>(y, hidden, nw, nw_dtype, w, H, N, eps, e, rp, st);
    return set_error(FD_EUNSUPPORTED, "the persistent SIMT QKV's registers do not hold M = %d", M);
  };
  using R2 = std::integral_constant<int, 2>;
  using R4 = std::integral_constant<int, 4>;
  using C1 = std::integral_constant<int, 1>;
  using C2 = std::integral_constant<int, 2>;
  using C4 = std::integral_constant<int, 4>;
  if (rows == 4) return cpl == 1 ? go(R4{}, C1{}) : cpl == 2 ? go(R4{}, C2{}) : go(R4{}, C4{});
  return cpl == 1 ? go(R2{}, C1{}) : cpl == 2 ? go(R2{}, C2{}) : go(R2{}, C4{});
}

// Whether the persistent SIMT QKV takes this launch: kind simt up to
// kQkvPxMaxM rows, kind dot up to kQkvPxDotMaxM (Llama-3-8B QKV, fp16: M = 1 /
// 2 / 4 10.8 / 10.9 / 11.2 us against 11.0 / 11.7 / 14.5 for the per-tile SIMT
// kernel; M = 5 / 6 12.4 / 12.5 against 13.4 / 13.5 for the MFMA kernel, which
// ties it at M = 8: 13.8).
constexpr int kQkvPxMaxM = 8;
constexpr int kQkvPxDotMaxM = 6;
inline bool qkv_px_takes(int M, int N, int H) {
  int rows = 0, cpl = 0;
  switch (M) {
#define FD_CASE(MM) \
  case MM: return qkv_px_shape<MM>(N, H, rows, cpl);
    FD_CASE(1) FD_CASE(2) FD_CASE(3) FD_CASE(4) FD_CASE(5) FD_CASE(6) FD_CASE(7) FD_CASE(8)
#undef FD_CASE
    default: return false;
  }
}

template <typename T>
int launch_qkv_px_m(int M, void* y, const void* hidden, const void* nw, int nw_dtype, const void* w, int H,
                    int N, float eps, const Epi& e, const Rope& rp, hipStream_t st) {
  switch (M) {
#define FD_CASE(MM) \
  case MM: return launch_qkv_px<T, MM>(y, hidden, nw, nw_dtype, w, H, N, eps, e, rp, st);
    FD_CASE(1) FD_CASE(2) FD_CASE(3) FD_CASE(4) FD_CASE(5) FD_CASE(6) FD_CASE(7) FD_CASE(8)
#undef FD_CASE
    default: return set_error(FD_EINVAL, "the persistent SIMT QKV takes M in [1, %d]", kQkvPxMaxM);
  }
}

template <typename T>
int launch_qkv_simt_m(int M, void* y, const void* hidden, const void* nw, int nw_dtype,
                      const void* w, int H, int N, float eps, const Epi& e, const Rope& rp,
                      hipStream_t st) {
  switch (M) {
#define FD_CASE(MM) \
  case MM: return launch_qkv_simt<T, MM>(y, hidden, nw, nw_dtype, w, H, N, eps, e, rp, st);
    FD_CASE(1) FD_CASE(2) FD_CASE(3) FD_CASE(4) FD_CASE(5) FD_CASE(6) FD_CASE(7) FD_CASE(8)
    FD_CASE(9) FD_CASE(10) FD_CASE(11) FD_CASE(12) FD_CASE(13) FD_CASE(14) FD_CASE(15)
    FD_CASE(16)
#undef FD_CASE
    default: return set_error(FD_EINVAL, "M must be in [1, 16]");
  }
}

template <typename T>
int launch_mlp_relayout(int M, void* mid, const void* normed, const void* wgu, int H, int I,
                        hipStream_t st) {
  // Four waves, each with two of its units in flight (M=8 at Llama-3-8B widths:
  // 39.3 us against 41.2 for eight waves and 39.8 for the one-unit loop).
  const int units = (H + kUnit - 1) / kUnit;
  const int nwv = units < 4 ? units : 4;
  const GateUpGrid gg = relayout_grid(I);
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(gg.blocks), dim3(nwv * kWave), 0, st, static_cast<T*>(mid),
                       static_cast<const T*>(normed), static_cast<const T*>(wgu), M, H, I, nullptr, FD_F32, 0.f,
                       RowSq{nullptr, 0}, gg.big);
  };
  // (the half-B form would spill here: 168 VGPRs and 20 bytes of scratch)
  if (gg.mix)
    launch(mlp_gate_up_relayout_kernel<T, true, false, false, false, true>);
  else
    launch(mlp_gate_up_relayout_kernel<T, true, false, false>);
  return FD_OK;
}

// The same gate/up from the raw hidden state, the RMSNorm inside the kernel
// (no row kernel first): its row sums from the producer (rq), or, with rq
// null, from a pass over hidden in the prologue.
template <typename T>
int launch_mlp_relayout_ss(int M, void* mid, const void* hidden, const void* nw, int nw_dtype,
                           const void* wgu, int H, int I, float eps, const RowSq* rq, hipStream_t st) {
  const int units = (H + kUnit - 1) / kUnit;
  const int nwv = units < kSsWaves ? units : kSsWaves;
  const size_t lds = relayout_ss_lds(H, kSsWaves);
  if (lds + (size_t)(kSsWaves * kWave + kSsWaves * 256) * 16 > kMaxLds)
    return set_error(FD_EUNSUPPORTED, "H too large for the norm weight's LDS stage");
  const GateUpGrid gg = relayout_grid(I);
  auto launch = [&](auto kernel) {
    if (!allow_lds(kernel, lds)) return set_error(FD_ELAUNCH, "cannot raise the LDS limit to %zu bytes", lds);
    hipLaunchKernelGGL(kernel, dim3(gg.blocks), dim3(nwv * kWave), lds, st, static_cast<T*>(mid),
                       static_cast<const T*>(hidden), static_cast<const T*>(wgu), M, H, I, nw, nw_dtype, eps,
                       rq ? *rq : RowSq{nullptr, 0}, gg.big);
    return (int)FD_OK;
  };
  if (gg.mix) {
    if (rq)
      return M <= 8 ? launch(mlp_gate_up_relayout_kernel<T, true, true, true, false, true>)
                    : launch(mlp_gate_up_relayout_kernel<T, true, true, false, false, true>);
    return M <= 8 ? launch(mlp_gate_up_relayout_kernel<T, true, true, true, true, true>)
                  : launch(mlp_gate_up_relayout_kernel<T, true, true, false, true, true>);
  }
  if (rq)
    return M <= 8 ? launch(mlp_gate_up_relayout_kernel<T, true, true, true>)
                  : launch(mlp_gate_up_relayout_kernel<T, true, true, false>);
  return M <= 8 ? launch(mlp_gate_up_relayout_kernel<T, true, true, true, true>)
                : launch(mlp_gate_up_relayout_kernel<T, true, true, false, true>);
}

// The kernel a call runs: a tile's row count names it (16 = MFMA, which needs
// kind=dot; 2, 4, 8 = SIMT); with no rows given, kind=dot runs MFMA from
// kMfmaMinM rows and SIMT below.
bool linear_uses_mfma(int64_t M, int kind, const Tile& t = Tile{}) {
  if (t.rows) return t.rows == 16;
  return kind == FD_KIND_DOT && M >= kMfmaMinM;
}

// Tile values the kernel that will run accepts (0 = default).
int check_tile(const Tile& t, int64_t M, int kind) {
  if (t.waves < 0 || t.waves > kMaxWaves) return set_error(FD_EINVAL, "waves must be in [0, 8]");
  if (t.rows == 16 && kind != FD_KIND_DOT)
    return set_error(FD_EINVAL, "16 rows per workgroup is the MFMA GEMV (kind=dot only)");
  if (linear_uses_mfma(M, kind, t)) {
    if (t.stages < 0 || t.stages > 3) return set_error(FD_EINVAL, "MFMA stages must be 0 to 3");
    if (t.waves != 0 && !dma_shape_ok(t.waves, t.stages ? t.stages : 2, (int)M))
      return set_error(FD_EINVAL, "MFMA waves must be 2, 4 or 8, within the LDS of a CU");
  } else {
    if (t.rows != 0 && t.rows != 2 && t.rows != 4 && t.rows != 8)
      return set_error(FD_EINVAL, "rows per workgroup must be 2, 4 or 8 (SIMT) or 16 (MFMA)");
    if (t.rows == 8 && M > 8) return set_error(FD_EINVAL, "8 SIMT rows per workgroup need M <= 8");
    if (t.stages < 0 || t.stages > 2)
      return set_error(FD_EINVAL, "SIMT stages must be 0 (default), 1 (per-tile) or 2 (persistent)");
  }
  return FD_OK;
}

// Launch the GEMV that fits the operands: the vector kernels need unit K
// stride, K % 8 == 0 and 16-byte aligned rows; anything else takes the generic one.
int linear_dispatch(void* y, const void* x, const void* w, const Epi& e, int64_t M, int64_t N,
                    int64_t K, int64_t sxm, int64_t sxk, int64_t swn, int64_t swk, int64_t sym,
                    int64_t syn, int kind, int act_dtype, hipStream_t st, const Tile& t = Tile{}) {
  const bool fast = K % 8 == 0 && swk == 1 && sxk == 1 && aligned16(w) && aligned16(x) &&
                    (N == 1 || swn % 8 == 0) && (M == 1 || sxm % 8 == 0) && N <= 0x7fffffffLL &&
                    K <= 0x7fffffffLL;
  if (!fast) {
    if (e.ss)
      return set_error(FD_EUNSUPPORTED, "row sums of squares need the vector GEMV's operand layout");
    if (N > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "N too large");
    if (act_dtype == FD_F16)
      hipLaunchKernelGGL(gemv_gen_kernel<f16>, dim3((unsigned)N), dim3(256), 0, st, (f16*)y,
                         (const f16*)x, (const f16*)w, (int)M, K, sxm, sxk, swn, swk, sym, syn, e);
    else
      hipLaunchKernelGGL(gemv_gen_kernel<bf16>, dim3((unsigned)N), dim3(256), 0, st, (bf16*)y,
                         (const bf16*)x, (const bf16*)w, (int)M, K, sxm, sxk, swn, swk, sym, syn,
                         e);
    return FD_OK;
  }
  const bool mfma = linear_uses_mfma(M, kind, t);
  if (e.ss && !mfma)
    return set_error(FD_EUNSUPPORTED, "row sums of squares come from the MFMA GEMV (kind=dot, M >= 5)");
  if (act_dtype == FD_F16) {
    if (mfma)
      return launch_mfma<f16>((int)M, y, x, w, (int)N, (int)K, sxm, swn, sym, syn, e, st, nullptr, &t);
    return launch_simt_m<f16>((int)M, y, x, w, (int)N, (int)K, sxm, swn, sym, syn, e, t, st);
  } else {
    if (mfma)
      return launch_mfma<bf16>((int)M, y, x, w, (int)N, (int)K, sxm, swn, sym, syn, e, st, nullptr, &t);
    return launch_simt_m<bf16>((int)M, y, x, w, (int)N, (int)K, sxm, swn, sym, syn, e, t, st);
  }
}

}  // namespace
}  // namespace fd

using namespace fd;

namespace fd {
namespace {

int linear_entry(void* y, const void* x, const void* w, const void* bias, int bias_dtype,
                 const void* row_add, int row_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                 int64_t sxk, int64_t swn, int64_t swk, int64_t sb, int64_t srm, int64_t srn,
                 int64_t sym, int64_t syn, const fd_tile* tile, int kind, int act_dtype,
                 float* ss_out, void* stream) {
  if (!check_act_dtype(act_dtype)) return FD_EINVAL;
  if (kind != FD_KIND_DOT && kind != FD_KIND_SIMT)
    return set_error(FD_EINVAL, "kind must be FD_KIND_DOT or FD_KIND_SIMT");
  if (M < 0 || N < 0 || K < 0) return set_error(FD_EINVAL, "negative size");
  if (M > 16) return set_error(FD_EINVAL, "linear_out only covers M <= 16");
  if (sxm < 0 || sxk < 0 || swn < 0 || swk < 0 || sb < 0 || srm < 0 || srn < 0 || sym < 0 ||
      syn < 0)
    return set_error(FD_EINVAL, "negative stride");
  if (bias && bias_dtype != act_dtype && bias_dtype != FD_F32)
    return set_error(FD_EINVAL, "bias must match x or be float32");
  if (row_add && !check_any_dtype(row_dtype, "row_dtype")) return FD_EINVAL;
  Tile t{0, 0, 0};
  if (tile) {
    t.rows = tile->rows;
    t.waves = tile->waves;
    t.stages = tile->stages;
    const int rc = check_tile(t, M, kind);
    if (rc != FD_OK) return rc;
  }
  if (M == 0 || N == 0) return FD_OK;
  // K = 0 reads neither operand (an empty torch tensor's pointer is null)
  if (!y || ((!x || !w) && K > 0)) return set_error(FD_EINVAL, "null pointer argument");
  Epi e;
  e.bias = bias;
  e.bias_dtype = bias_dtype;
  e.sb = sb;
  e.row = row_add;
  e.row_dtype = row_dtype;
  e.srm = srm;
  e.srn = srn;
  e.ss = ss_out;
  const int rc = linear_dispatch(y, x, w, e, M, N, K, sxm, sxk, swn, swk, sym, syn, kind,
                                 act_dtype, static_cast<hipStream_t>(stream), t);
  if (rc != FD_OK) return rc;
  return check_launch();
}

}  // namespace
}  // namespace fd

extern "C" int fd_linear_tiled(void* y, const void* x, const void* w, const void* bias,
                               int bias_dtype, const void* row_add, int row_dtype, int64_t M,
                               int64_t N, int64_t K, int64_t sxm, int64_t sxk, int64_t swn,
                               int64_t swk, int64_t sb, int64_t srm, int64_t srn, int64_t sym,
                               int64_t syn, const fd_tile* tile, int kind, int act_dtype,
                               void* stream) {
  return linear_entry(y, x, w, bias, bias_dtype, row_add, row_dtype, M, N, K, sxm, sxk, swn, swk, sb,
                      srm, srn, sym, syn, tile, kind, act_dtype, nullptr, stream);
}

extern "C" int fd_linear_sumsq(void* y, const void* x, const void* w, const void* bias,
                               int bias_dtype, const void* row_add, int row_dtype, int64_t M,
                               int64_t N, int64_t K, int64_t sxm, int64_t sxk, int64_t swn,
                               int64_t swk, int64_t sb, int64_t srm, int64_t srn, int64_t sym,
                               int64_t syn, int kind, int act_dtype, float* ss_out, void* stream) {
  if (!ss_out) return set_error(FD_EINVAL, "null pointer argument");
  if (!aligned16(ss_out)) return set_error(FD_EUNSUPPORTED, "ss_out must be 16-byte aligned");
  if (!(kind == FD_KIND_DOT && M >= kMfmaMinM && M <= 16))
    return set_error(FD_EUNSUPPORTED, "row sums of squares come from the MFMA GEMV (kind=dot, M >= 5)");
  return linear_entry(y, x, w, bias, bias_dtype, row_add, row_dtype, M, N, K, sxm, sxk, swn, swk, sb,
                      srm, srn, sym, syn, nullptr, kind, act_dtype, ss_out, stream);
}

extern "C" int fd_linear(void* y, const void* x, const void* w, const void* bias, int bias_dtype,
                         const void* row_add, int row_dtype, int64_t M, int64_t N, int64_t K,
                         int64_t sxm, int64_t sxk, int64_t swn, int64_t swk, int64_t sb,
                         int64_t srm, int64_t srn, int64_t sym, int64_t syn, int kind,
                         int act_dtype, void* stream) {
  return fd_linear_tiled(y, x, w, bias, bias_dtype, row_add, row_dtype, M, N, K, sxm, sxk, swn,
                         swk, sb, srm, srn, sym, syn, nullptr, kind, act_dtype, stream);
}

namespace fd {
namespace {

int mlp_check(void* mid, const void* hidden, const void* norm_w, int norm_w_dtype,
              const void* w_gate_up, int64_t M, int64_t H, int64_t I, float eps, int kind,
              int act_dtype) {
  if (!check_act_dtype(act_dtype) || !check_any_dtype(norm_w_dtype, "norm_w_dtype"))
    return FD_EINVAL;
  if (kind != FD_KIND_DOT && kind != FD_KIND_SIMT)
    return set_error(FD_EINVAL, "kind must be FD_KIND_DOT or FD_KIND_SIMT");
  if (M < 0 || M > 16) return set_error(FD_EINVAL, "M must be in [0, 16]");
  if (H <= 0 || I <= 0) return set_error(FD_EINVAL, "H and I must be positive");
  if (!(eps >= 0.f) || eps == INFINITY) return set_error(FD_EINVAL, "eps must be a finite value >= 0");
  if (M == 0) return FD_OK;
  if (!mid || !hidden || !norm_w || !w_gate_up) return set_error(FD_EINVAL, "null pointer argument");
  if (H % 8 != 0 || I % 8 != 0)
    return set_error(FD_EUNSUPPORTED, "H and I must be multiples of 8");
  if (H > 0x7fffffffLL || 2 * I > 0x7fffffffLL) return set_error(FD_EUNSUPPORTED, "too large");
  if (!aligned16(mid) || !aligned16(hidden) || !aligned16(norm_w) || !aligned16(w_gate_up))
    return set_error(FD_EUNSUPPORTED, "operands must be 16-byte aligned");
  return FD_OK;
}

bool mlp_mfma(int64_t M, int kind) { return kind == FD_KIND_DOT && M >= kMfmaMinM; }
// Whether the MFMA gate/up normalises x inside the kernel with no producer
// sums: up to 8 rows, while the norm weight's LDS stage fits (H up to about
// 35,000); otherwise the MFMA form runs a row kernel into `normed` first.
bool mlp_fold(int64_t M, int64_t H) {
  return M <= 8 && relayout_ss_lds((int)H, kSsWaves) + (size_t)(kSsWaves * kWave + kSsWaves * 256) * 16 <= kMaxLds;
}
// Whether the gate/up launch of this call needs the [M, H] `normed` buffer.
bool mlp_needs_normed(int64_t M, int64_t H, int kind) { return mlp_mfma(M, kind) && !mlp_fold(M, H); }

int mlp_gate_up(void* mid, void* normed, const void* hidden, const void* norm_w, int norm_w_dtype,
                const void* w_gate_up, int64_t M, int64_t H, int64_t I, float eps, int kind,
                int act_dtype, hipStream_t st, const RowSq* rq = nullptr) {
  int rc;
  if (rq || (mlp_mfma(M, kind) && mlp_fold(M, H))) {
    // MFMA form, normalised inside the kernel: row sums from the producer, or from
    // a pass over x (up to 8 rows; from 9 its registers would spill: 168 VGPRs
    // and 12 bytes of scratch), one launch instead of the row kernel + gate/up
    // (Llama-3-8B widths, M=8: whole MLP 69.3 -> 66.3 us eager)
    rc = act_dtype == FD_F16
             ? launch_mlp_relayout_ss<f16>((int)M, mid, hidden, norm_w, norm_w_dtype, w_gate_up, (int)H,
                                           (int)I, eps, rq, st)
             : launch_mlp_relayout_ss<bf16>((int)M, mid, hidden, norm_w, norm_w_dtype, w_gate_up, (int)H,
                                            (int)I, eps, rq, st);
  } else if (mlp_needs_normed(M, H, kind)) {
    // The relayout kernel (register loads, 16 gate and 16 up rows per workgroup
    // against one B tile), not the DMA form: Llama-3-8B widths, M=8, whole MLP
    // 63.5 us against 72.9 for DMA workgroups of the same two tiles, 69.9 for
    // DMA tiles of 8 gate + 8 up rows, 77.7 for those with the norm folded in.
    rc = rms_rows(normed, hidden, norm_w, norm_w_dtype, M, H, eps, act_dtype, st);
    if (rc != FD_OK) return rc;
    rc = act_dtype == FD_F16
             ? launch_mlp_relayout<f16>((int)M, mid, normed, w_gate_up, (int)H, (int)I, st)
             : launch_mlp_relayout<bf16>((int)M, mid, normed, w_gate_up, (int)H, (int)I, st);
  } else {
    rc = act_dtype == FD_F16
             ? launch_mlp_simt_m<f16>((int)M, mid, hidden, norm_w, norm_w_dtype, w_gate_up,
                                      (int)H, (int)I, eps, st)
             : launch_mlp_simt_m<bf16>((int)M, mid, hidden, norm_w, norm_w_dtype, w_gate_up,
                                       (int)H, (int)I, eps, st);
  }
  if (rc != FD_OK) return rc;
  return check_launch();
}

}  // namespace
}  // namespace fd

extern "C" int fd_mlp_gate_up(void* mid, void* normed, const void* hidden, const void* norm_w,
                              int norm_w_dtype, const void* w_gate_up, int64_t M, int64_t H,
                              int64_t I, float eps, int kind, int act_dtype, void* stream) {
  int rc = mlp_check(mid, hidden, norm_w, norm_w_dtype, w_gate_up, M, H, I, eps, kind, act_dtype);
  if (rc != FD_OK || M == 0) return rc;
  if (mlp_needs_normed(M, H, kind)) {
    if (!normed) return set_error(FD_EINVAL, "kind=dot with M >= 9 needs the normed buffer");
    if (!aligned16(normed)) return set_error(FD_EUNSUPPORTED, "operands must be 16-byte aligned");
  }
  return mlp_gate_up(mid, normed, hidden, norm_w, norm_w_dtype, w_gate_up, M, H, I, eps, kind,
                     act_dtype, static_cast<hipStream_t>(stream));
}

namespace fd {
namespace {

int post_attn_mlp_entry(void* y, void* mid, const void* hidden, const void* norm_w, int norm_w_dtype,
                        const void* w_gate_up, const void* w_down, int64_t M, int64_t H, int64_t I,
                        float eps, int kind, int act_dtype, const RowSq* rq, float* ss_out,
                        void* stream) {
  int rc = mlp_check(mid, hidden, norm_w, norm_w_dtype, w_gate_up, M, H, I, eps, kind, act_dtype);
  if (rc != FD_OK || M == 0) return rc;
  if (!y || !w_down) return set_error(FD_EINVAL, "null pointer argument");
  rc = check_mlp_buffers(y, mid, hidden, M, H, I, 2);
  if (rc != FD_OK) return rc;
  if (!aligned16(y) || !aligned16(w_down))
    return set_error(FD_EUNSUPPORTED, "operands must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // y doubles as the normed buffer of the MFMA form: the down projection, which
  // writes y, runs after the gate/up launch has consumed it.
  rc = mlp_gate_up(mid, y, hidden, norm_w, norm_w_dtype, w_gate_up, M, H, I, eps, kind,
                   act_dtype, st, rq);
  if (rc != FD_OK) return rc;
  Epi e;
  e.bias = nullptr;
  e.bias_dtype = act_dtype;
  e.sb = 0;
  e.row = hidden;
  e.row_dtype = act_dtype;
  e.srm = H;
  e.srn = 1;
  e.ss = ss_out;
  rc = linear_dispatch(y, mid, w_down, e, M, H, I, I, 1, I, 1, H, 1, kind, act_dtype, st);
  if (rc != FD_OK) return rc;
  return check_launch();
}

}  // namespace
}  // namespace fd

extern "C" int fd_post_attn_mlp(void* y, void* mid, const void* hidden, const void* norm_w,
                                int norm_w_dtype, const void* w_gate_up, const void* w_down,
                                int64_t M, int64_t H, int64_t I, float eps, int kind,
                                int act_dtype, void* stream) {
  return post_attn_mlp_entry(y, mid, hidden, norm_w, norm_w_dtype, w_gate_up, w_down, M, H, I, eps, kind,
                             act_dtype, nullptr, nullptr, stream);
}

extern "C" int fd_post_attn_mlp_sumsq(void* y, void* mid, const void* hidden, const void* norm_w,
                                      int norm_w_dtype, const void* w_gate_up, const void* w_down,
                                      int64_t M, int64_t H, int64_t I, float eps, int kind,
                                      int act_dtype, const float* ss_in, int64_t ss_tiles,
                                      float* ss_out, void* stream) {
  const int rc = check_sumsq(kind == FD_KIND_DOT && M >= kMfmaMinM, ss_in, ss_tiles, H, ss_out);
  if (rc != FD_OK) return rc;
  const RowSq rq{ss_in, (int)ss_tiles};
  return post_attn_mlp_entry(y, mid, hidden, norm_w, norm_w_dtype, w_gate_up, w_down, M, H, I, eps, kind,
                             act_dtype, ss_in ? &rq : nullptr, ss_out, stream);
}

// ---------------------------------------------------------------------------
// fd_post_attn_mlp_noalloc: the same MLP with `mid` in library-owned device
// memory, for callers that cannot allocate (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).

namespace fd {
namespace {

// The [M, I] SwiGLU rows of one call: M * I * 2 bytes, 458,752 at Llama-3-8B
// widths and M = 16. Each GPU holds one copy for the life of the process.
constexpr int64_t kScratchBytes = int64_t(1) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `device`. Host code must never pass the
// array's own name to a kernel or a copy (it names a host-side stand-in), so
// the address is looked up once per device, with that device current, and
// kept. Restores the caller's current device.
int scratch_ptr(int device, void** out) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(FD_EUNSUPPORTED, "device %d: the library scratch covers devices 0..%d", device,
                     kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return set_error(FD_ELAUNCH, "hipGetDevice failed");
    if (prev != device && hipSetDevice(device) != hipSuccess)
      return set_error(FD_ELAUNCH, "hipSetDevice(%d) failed", device);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (prev != device) (void)hipSetDevice(prev);
    if (e != hipSuccess || !p)
      return set_error(FD_ELAUNCH, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return FD_OK;
}

}  // namespace
}  // namespace fd

extern "C" int fd_init(void) {
  using namespace fd;
  int count = 0;
  const hipError_t e = hipGetDeviceCount(&count);
  if (e == hipErrorNoDevice || (e == hipSuccess && count == 0)) {
    (void)hipGetLastError();  // no GPU: nothing to set up
    return FD_OK;
  }
  if (e != hipSuccess) return set_error(FD_ELAUNCH, "hipGetDeviceCount failed: %s", hipGetErrorString(e));
  for (int d = 0; d < count && d < kMaxDevices; ++d) {
    void* p = nullptr;
    const int rc = scratch_ptr(d, &p);
    if (rc != FD_OK) return rc;
  }
  return FD_OK;
}

extern "C" int fd_post_attn_mlp_noalloc(void* y, const void* hidden, const void* norm_w,
                                        int norm_w_dtype, const void* w_gate_up,
                                        const void* w_down, int64_t M, int64_t H, int64_t I,
                                        float eps, int kind, int act_dtype, void* stream) {
  using namespace fd;
  if (!check_act_dtype(act_dtype)) return FD_EINVAL;
  if (M < 0 || M > 16) return set_error(FD_EINVAL, "M must be in [0, 16]");
  if (H <= 0 || I <= 0) return set_error(FD_EINVAL, "H and I must be positive");
  if (M * I * 2 > kScratchBytes)
    return set_error(FD_EINVAL, "M*I*2 = %lld bytes exceeds the %lld-byte library scratch",
                     (long long)(M * I * 2), (long long)kScratchBytes);
  if (M == 0) return FD_OK;
  int device = 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const hipError_t e = st ? hipStreamGetDevice(st, &device) : hipGetDevice(&device);
  if (e != hipSuccess) return set_error(FD_ELAUNCH, "cannot find the stream's device");
  void* mid = nullptr;
  const int rc = scratch_ptr(device, &mid);
  if (rc != FD_OK) return rc;
  return fd_post_attn_mlp(y, mid, hidden, norm_w, norm_w_dtype, w_gate_up, w_down, M, H, I, eps,
                          kind, act_dtype, stream);
}

namespace fd {
namespace {

int pre_attn_qkv_entry(void* y, void* normed, const void* hidden, const void* norm_w, int norm_w_dtype,
                       const void* w_qkv, const void* bias, int bias_dtype, const void* cos, const void* sin,
                       int cs_dtype, int64_t cs_row_stride, int64_t M, int64_t H, int64_t N, int64_t rope_cols,
                       int64_t head_dim, float eps, int kind, int act_dtype, const RowSq* rq, void* stream) {
  if (kind != FD_KIND_DOT && kind != FD_KIND_SIMT)
    return set_error(FD_EINVAL, "kind must be FD_KIND_DOT or FD_KIND_SIMT");
  const bool mfma = mlp_mfma(M, kind);
  Epi e;
  Rope rp;
  bool empty = false;
  // the MFMA form folds the RMSNorm in: `normed` is not used at any M
  const int checked = qkv_prepare(y, normed, hidden, norm_w, norm_w_dtype, w_qkv, bias, bias_dtype,
                                  cos, sin, cs_dtype, cs_row_stride, M, H, N, rope_cols, head_dim,
                                  eps, act_dtype, false, e, rp, empty);
  if (checked != FD_OK || empty) return checked;
  if (H % 8 != 0) return set_error(FD_EUNSUPPORTED, "H must be a multiple of 8");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc;
  if (M <= (kind == FD_KIND_SIMT ? kQkvPxMaxM : kQkvPxDotMaxM) && qkv_px_takes((int)M, (int)N, (int)H)) {
    rc = act_dtype == FD_F16
             ? launch_qkv_px_m<f16>((int)M, y, hidden, norm_w, norm_w_dtype, w_qkv, (int)H, (int)N, eps, e, rp, st)
             : launch_qkv_px_m<bf16>((int)M, y, hidden, norm_w, norm_w_dtype, w_qkv, (int)H, (int)N, eps, e, rp, st);
    if (rc != FD_OK) return rc;
  } else if (mfma) {  // one launch: the RMSNorm folded into the MFMA kernel
    rp.tiles = (int)(rope_cols / 16);
    FoldNorm fn{norm_w, norm_w_dtype, eps};
    if (rq) fn.sq = *rq;
    rc = act_dtype == FD_F16
             ? launch_mfma<f16>((int)M, y, hidden, w_qkv, (int)N, (int)H, H, H, N, 1, e, st, &rp, nullptr, &fn)
             : launch_mfma<bf16>((int)M, y, hidden, w_qkv, (int)N, (int)H, H, H, N, 1, e, st, &rp, nullptr, &fn);
    if (rc != FD_OK) return rc;
  } else {
    rc = act_dtype == FD_F16
             ? launch_qkv_simt_m<f16>((int)M, y, hidden, norm_w, norm_w_dtype, w_qkv, (int)H,
                                      (int)N, eps, e, rp, st)
             : launch_qkv_simt_m<bf16>((int)M, y, hidden, norm_w, norm_w_dtype, w_qkv, (int)H,
                                       (int)N, eps, e, rp, st);
    if (rc != FD_OK) return rc;
  }
  return check_launch();
}

}  // namespace
}  // namespace fd

extern "C" int fd_pre_attn_qkv(void* y, void* normed, const void* hidden, const void* norm_w,
                               int norm_w_dtype, const void* w_qkv, const void* bias,
                               int bias_dtype, const void* cos, const void* sin, int cs_dtype,
                               int64_t cs_row_stride, int64_t M, int64_t H, int64_t N,
                               int64_t rope_cols, int64_t head_dim, float eps, int kind,
                               int act_dtype, void* stream) {
  return pre_attn_qkv_entry(y, normed, hidden, norm_w, norm_w_dtype, w_qkv, bias, bias_dtype, cos, sin,
                            cs_dtype, cs_row_stride, M, H, N, rope_cols, head_dim, eps, kind, act_dtype,
                            nullptr, stream);
}

extern "C" int fd_pre_attn_qkv_sumsq(void* y, const void* hidden, const void* norm_w, int norm_w_dtype,
                                     const void* w_qkv, const void* bias, int bias_dtype, const void* cos,
                                     const void* sin, int cs_dtype, int64_t cs_row_stride, int64_t M,
                                     int64_t H, int64_t N, int64_t rope_cols, int64_t head_dim, float eps,
                                     int kind, int act_dtype, const float* ss_in, int64_t ss_tiles,
                                     void* stream) {
  if (!ss_in) return set_error(FD_EINVAL, "null pointer argument");
  const int rc = check_sumsq(kind == FD_KIND_DOT && M >= kMfmaMinM, ss_in, ss_tiles, H, nullptr);
  if (rc != FD_OK) return rc;
  const RowSq rq{ss_in, (int)ss_tiles};
  return pre_attn_qkv_entry(y, nullptr, hidden, norm_w, norm_w_dtype, w_qkv, bias, bias_dtype, cos, sin,
                            cs_dtype, cs_row_stride, M, H, N, rope_cols, head_dim, eps, kind, act_dtype, &rq,
                            stream);
}
