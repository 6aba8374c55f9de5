// SPDX-License-Identifier: Apache-2.0
// Hyena operator chain of one StripedHyena2 block on gfx950:
//
//   P [L, 3W] --short FIR (k=3, per column)--> (x2, x1, v) per channel
//   u = x1 * v
//   HCS: y = x2 * FIR_7(u)            grouped cross-correlation, groups G
//   HCM: y = x2 * (conv_128(u) + D*u) grouped causal convolution
//   HCL: y = x2 * (sum_m R_m s_m + D*u),  s_m <- p_m s_m + u   (p = exp(logp))
//
// Semantics follow evo.cpp `src/cpu/model.cpp:426-453` (FIR with explicit
// history, tap order) and `:546-605` (mixer), F32 arithmetic. The short FIR
// and the gates are recomputed inside each kernel straight from P, so the
// [L, W] intermediates x2 and u never go to HBM.
//
// HCL is evaluated as a chunked scan, exact in exact arithmetic: chunks of
// kChunk rows run in parallel from a zero state (phase 1 keeps only each
// chunk's final state), a short carry pass turns those into the true state at
// every chunk start (s_in[g+1] = p^len * s_in[g] + s_loc[g]), and phase 3
// rescans each chunk from its true state and writes y. One thread owns one
// channel and keeps its 16 modal states in registers.
#include "common.hpp"
#include "ops.hpp"

#include <mutex>
#include <type_traits>

namespace evo::hip {
namespace {

constexpr int kChannels = 64;    // channels per block (one wave)
constexpr int kChunk = 128;      // HCL rows per chunk
constexpr int kMaxState = 16;
constexpr int kMaxShort = 8;

// Column of projection stream s (0 = x2, 1 = x1, 2 = v) of channel c. The
// reference layout interleaves the streams (3c + s); the planar layout keeps
// each stream contiguous (s * W + c), so a wave's 64 channels of one stream
// are one 128-byte (BF16) segment. `planar` is W for the planar layout and 0
// for the interleaved one. The short FIR history uses the same columns.
__device__ inline size_t pcol(size_t c, int s, size_t planar) {
  return planar != 0 ? static_cast<size_t>(s) * planar + c : 3 * c + static_cast<size_t>(s);
}

// Reads column `col` of P at row t (t may be negative: the short history holds
// rows -(short_len-1)..-1, oldest first).
template <typename T>
__device__ inline float p_at(const T *P, const float *short_history,
                             size_t cols3, size_t short_hist_rows, long t,
                             size_t col) {
  if (t >= 0)
    return load_act(P, static_cast<size_t>(t) * cols3 + col);
  const long h = static_cast<long>(short_hist_rows) + t;
  if (short_history == nullptr || h < 0)
    return 0.0F;
  return short_history[static_cast<size_t>(h) * cols3 + col];
}

// Short FIR of column `col` at row t: cross-correlation, tap j multiplies
// row t - (k-1) + j, accumulated oldest first.
template <typename T>
__device__ inline float short_fir(const T *P, const float *short_history,
                                  const float *taps, int k, size_t cols3,
                                  long t, size_t col) {
  float total = 0.0F;
  for (int j = 0; j < k; ++j)
    total += p_at(P, short_history, cols3, k - 1, t - (k - 1) + j, col) * taps[j];
  return total;
}

template <typename T>
__device__ inline void gates(const T *P, const float *short_history,
                             const float (&taps)[3][kMaxShort], int k,
                             size_t cols3, size_t planar, long t, size_t c,
                             float *x2, float *u) {
  *x2 = short_fir(P, short_history, taps[0], k, cols3, t, pcol(c, 0, planar));
  const float x1 = short_fir(P, short_history, taps[1], k, cols3, t, pcol(c, 1, planar));
  const float v = short_fir(P, short_history, taps[2], k, cols3, t, pcol(c, 2, planar));
  *u = x1 * v;
}

__device__ inline void load_short_taps(const uint16_t *filter, int k, size_t c,
                                       float (&taps)[3][kMaxShort]) {
  for (int s = 0; s < 3; ++s)
    for (int j = 0; j < kMaxShort; ++j)
      taps[s][j] = j < k ? bf16_to_f32(filter[(3 * c + s) * k + j]) : 0.0F;
}

// ---- HCL row streaming. Each thread keeps the last kWin rows of its three
// projection columns in registers, so every row of P is loaded once; rows
// are fetched kBatch at a time to keep that many loads in flight. The short
// FIR taps are stored right-aligned in a kWin-wide window (zeros in front),
// which keeps the oldest-first accumulation order of the reference.
constexpr int kBatch = 8;

template <int kWin>
__device__ inline void load_window_taps(const uint16_t *filter, int k, size_t c,
                                        float (&taps)[3][kWin]) {
#pragma unroll
  for (int s = 0; s < 3; ++s)
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
      const int j = i - (kWin - k);  // tap index of window slot i
      taps[s][i] = j >= 0 ? bf16_to_f32(filter[(3 * c + s) * k + j]) : 0.0F;
    }
}

template <typename T, int kWin>
struct RowStream {
  float win[3][kWin];  // win[s][kWin-1] = current row
  float taps[3][kWin];

  // Fills the window with the rows before t0 (history rows when t0 is 0).
  __device__ void prime(const T *P, const float *short_history, int k,
                        size_t cols3, size_t planar, long t0, size_t c) {
#pragma unroll
    for (int i = 0; i < kWin - 1; ++i) {
      const long t = t0 - (kWin - 1) + i;
      // Rows older than the filter reach only meet zero taps.
      const bool used = t >= t0 - (k - 1);
#pragma unroll
      for (int s = 0; s < 3; ++s)
        win[s][i + 1] = used ? p_at(P, short_history, cols3, k - 1, t, pcol(c, s, planar)) : 0.0F;
    }
  }
  // Shifts in one row and returns the FIR outputs of its three columns.
  __device__ void push(const float (&row)[3], float (&fir)[3]) {
#pragma unroll
    for (int s = 0; s < 3; ++s) {
#pragma unroll
      for (int i = 0; i < kWin - 1; ++i)
        win[s][i] = win[s][i + 1];
      win[s][kWin - 1] = row[s];
      float total = 0.0F;
#pragma unroll
      for (int i = 0; i < kWin; ++i)
        total += win[s][i] * taps[s][i];
      fir[s] = total;
    }
  }
};

// Loads rows [t, t + kB) (clipped to t1) of the channel's 3 columns.
template <typename T, int kB>
__device__ inline void load_batch(const T *P, size_t cols3, size_t planar, size_t t,
                                  size_t t1, size_t c, float (&rows)[kB][3]) {
  // Rows at or past t1 lie beyond the resource bound and read 0.
  const uint32_t row_bytes = static_cast<uint32_t>(cols3 * sizeof(T));
  const auto resource = buffer_resource(P + t * cols3, static_cast<uint32_t>(t1 - t) * row_bytes);
  uint32_t column[3];
#pragma unroll
  for (int s = 0; s < 3; ++s)
    column[s] = static_cast<uint32_t>(pcol(c, s, planar) * sizeof(T));
#pragma unroll
  for (int b = 0; b < kB; ++b)
#pragma unroll
    for (int s = 0; s < 3; ++s)
      rows[b][s] = buffer_act<T>(resource, column[s], b * row_bytes);
}

// ---- HCL phase 1: final local state of every chunk from a zero start.
template <typename T, int kWin>
__global__ __launch_bounds__(kChannels) void hcl_chunk_state_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len, size_t L,
    size_t W, size_t planar, const float *__restrict__ poles, int S, float *__restrict__ chunk_state) {
  const size_t c = blockIdx.x * static_cast<size_t>(kChannels) + threadIdx.x;
  if (c >= W)
    return;
  const size_t g = blockIdx.y;
  const size_t t0 = g * kChunk, t1 = min(L, t0 + kChunk);
  const size_t cols3 = 3 * W;
  RowStream<T, kWin> stream;
  load_window_taps(short_filter, short_len, c, stream.taps);
  stream.prime(P, short_history, short_len, cols3, planar, static_cast<long>(t0), c);
  float p[kMaxState], s[kMaxState];
#pragma unroll
  for (int m = 0; m < kMaxState; ++m) {
    p[m] = m < S ? poles[c * S + m] : 0.0F;
    s[m] = 0.0F;
  }
  for (size_t t = t0; t < t1; t += kBatch) {
    float rows[kBatch][3];
    load_batch(P, cols3, planar, t, t1, c, rows);
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (t + b >= t1)
        break;
      float fir[3];
      stream.push(rows[b], fir);
      const float u = fir[1] * fir[2];
#pragma unroll
      for (int m = 0; m < kMaxState; ++m)
        s[m] = p[m] * s[m] + u;
    }
  }
#pragma unroll
  for (int m = 0; m < kMaxState; ++m)
    if (m < S)
      chunk_state[(g * S + m) * W + c] = s[m];
}

// ---- HCL phase 2: chunk-start states (in place) and the final state.
__global__ void hcl_carry_kernel(float *__restrict__ chunk_state, size_t G,
                                 size_t L, size_t W, int S,
                                 const float *__restrict__ poles,
                                 float *__restrict__ modal_state) {
  const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (i >= W * S)
    return;
  const size_t m = i / W, c = i % W;
  const float p = poles[c * S + m];
  // p^kChunk by repeated squaring (kChunk is a power of two).
  float full = p;
  for (int e = 1; e < kChunk; e <<= 1)
    full *= full;
  float state = modal_state != nullptr ? modal_state[c * S + m] : 0.0F;
  // Chunk states are loaded 16 at a time ahead of the serial combine, so
  // the loads overlap instead of forming a load -> store chain per chunk.
  constexpr int kAhead = 16;
  for (size_t g0 = 0; g0 < G; g0 += kAhead) {
    float local[kAhead];
#pragma unroll
    for (int q = 0; q < kAhead; ++q)
      local[q] = g0 + q < G ? chunk_state[((g0 + q) * S + m) * W + c] : 0.0F;
#pragma unroll
    for (int q = 0; q < kAhead; ++q) {
      const size_t g = g0 + q;
      if (g >= G)
        continue;
      chunk_state[(g * S + m) * W + c] = state;
      const size_t len = min(L - g * kChunk, static_cast<size_t>(kChunk));
      float power = full;
      if (len != static_cast<size_t>(kChunk)) {
        power = 1.0F;
        for (size_t e = 0; e < len; ++e)
          power *= p;
      }
      state = power * state + local[q];
    }
  }
  if (modal_state != nullptr)
    modal_state[c * S + m] = state;
}

// ---- HCL phase 3: rescan each chunk from its true start state.
template <typename T, typename O, int kWin>
__global__ __launch_bounds__(kChannels) void hcl_output_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len, size_t L,
    size_t W, size_t planar, const float *__restrict__ poles,
    const float *__restrict__ residues, const float *__restrict__ direct,
    int S, const float *__restrict__ chunk_state, O out) {
  const size_t c = blockIdx.x * static_cast<size_t>(kChannels) + threadIdx.x;
  if (c >= W)
    return;
  const size_t g = blockIdx.y;
  const size_t t0 = g * kChunk, t1 = min(L, t0 + kChunk);
  const size_t cols3 = 3 * W;
  RowStream<T, kWin> stream;
  load_window_taps(short_filter, short_len, c, stream.taps);
  stream.prime(P, short_history, short_len, cols3, planar, static_cast<long>(t0), c);
  float p[kMaxState], r[kMaxState], s[kMaxState];
#pragma unroll
  for (int m = 0; m < kMaxState; ++m) {
    p[m] = m < S ? poles[c * S + m] : 0.0F;
    r[m] = m < S ? residues[c * S + m] : 0.0F;
    s[m] = m < S ? chunk_state[(g * S + m) * W + c] : 0.0F;
  }
  const float d = direct[c];
  for (size_t t = t0; t < t1; t += kBatch) {
    float rows[kBatch][3];
    load_batch(P, cols3, planar, t, t1, c, rows);
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (t + b >= t1)
        break;
      float fir[3];
      stream.push(rows[b], fir);
      const float x2 = fir[0], u = fir[1] * fir[2];
      float modal = 0.0F;
#pragma unroll
      for (int m = 0; m < kMaxState; ++m) {
        s[m] = p[m] * s[m] + u;
        modal += r[m] * s[m];
      }
      put_nt(out, (t + b) * W + c, x2 * (modal + d * u));
    }
  }
}

// ---- HCS / HCM: grouped FIR over u with an explicit [k-1, W] history.
// Block: 64 channels x kTile rows. u for rows [t0-(k-1), t0+kTile) is staged
// in LDS (computed from P), then each lane produces its channel's outputs.
template <int kTile>
__device__ inline void stage_u(const void *, int) {}

template <typename T, typename O, int kTile, int kMaxTaps>
__global__ __launch_bounds__(256) void hyena_fir_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len,
    const float *__restrict__ inner_history, const float *__restrict__ filter,
    size_t groups, int k, int causal, const float *__restrict__ direct,
    size_t L, size_t W, size_t planar, O out) {
  extern __shared__ float smem[];
  float *u_s = smem;                                  // [(k-1) + kTile][64]
  float *x2_s = smem + (kMaxTaps - 1 + kTile) * 64;   // [kTile][64]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const size_t c = blockIdx.x * static_cast<size_t>(kChannels) + lane;
  const long t0 = static_cast<long>(blockIdx.y) * kTile;
  const bool valid = c < W;
  const int hist = k - 1;
  float taps[3][kMaxShort];
  if (valid)
    load_short_taps(short_filter, short_len, c, taps);
  const size_t cols3 = 3 * W;
  const long rows_total = hist + kTile;
  for (long r = wave; r < rows_total; r += 4) {
    const long t = t0 - hist + r;
    float x2 = 0.0F, u = 0.0F;
    if (valid && t < static_cast<long>(L)) {
      if (t >= 0) {
        gates(P, short_history, taps, short_len, cols3, planar, t, c, &x2, &u);
      } else {
        const long h = static_cast<long>(hist) + t;
        u = (inner_history != nullptr && h >= 0) ? inner_history[h * W + c] : 0.0F;
      }
    }
    u_s[r * 64 + lane] = u;
    if (r >= hist)
      x2_s[(r - hist) * 64 + lane] = x2;
  }
  __syncthreads();
  if (!valid)
    return;
  const size_t group = c / (W / groups);
  const float *h = filter + group * k;
  const float d = direct != nullptr ? direct[c] : 0.0F;
  for (int r = wave; r < kTile; r += 4) {
    const long t = t0 + r;
    if (t >= static_cast<long>(L))
      break;
    // Output row r reads u rows r .. r + hist of the staged window (oldest
    // first). Cross-correlation pairs the oldest with tap 0; causal
    // convolution with tap k-1.
    float total = 0.0F;
    for (int old = 0; old < hist; ++old) {
      const int tap = causal ? k - 1 - old : old;
      total += u_s[(r + old) * 64 + lane] * h[tap];
    }
    const float current = u_s[(r + hist) * 64 + lane];
    total += current * h[causal ? 0 : hist];
    if (direct != nullptr)
      total += d * current;
    put(out, static_cast<size_t>(t) * W + c, x2_s[r * 64 + lane] * total);
  }
}

// ---- Short grouped FIR (k <= 8, HCS) as a row stream on the VALU.
// Each lane owns two adjacent channels: their six interleaved projection
// columns are 12 (BF16) or 24 (F32) contiguous bytes of a row, and the two
// outputs are one packed 32-bit store per plane. A wave streams a segment of
// 64 or 128 rows (kStreamRows, kStreamMaxRows); it starts kLead rows early
// so that its short-FIR window and its FIR window of u are full when the
// segment begins (the lead rows are recomputed, not stored). Both windows
// hold their taps right-aligned with zeros in front, so every sum runs oldest
// first as in the reference; with kWin == short_len and kTaps == k there are
// no zero taps. Rows are fetched
// in batches of kStreamBatch with the next batch in flight while the current
// one is evaluated. Stores go through a buffer resource bounded to the
// segment, so rows past the sequence end are dropped by the hardware, and
// are non-temporal: the outputs are never re-read here, and streaming them
// past the L2 keeps it for the projection rows (-23 % kernel time on the 7B
// shape).
// Segment length: 64 rows, doubled to 128 when the grid keeps at least
// kStreamMinBlocks blocks (two per CU): longer segments recompute fewer lead
// rows (7B, L = 8192: 58 -> 54 us; 256 rows measured no better).
constexpr int kStreamRows = 64;
constexpr int kStreamMaxRows = 128;
constexpr unsigned kStreamMinBlocks = 512;
constexpr int kStreamBatch = 4;
constexpr int kStreamWaves = 4;              // waves per block
constexpr int kStreamChannels = kStreamWaves * 64 * 2;
constexpr int kStreamStore = 2;              // buffer store cache policy: nt

// Six projection values (channel c: x2, x1, v; channel c + 1: x2, x1, v) of
// one row as 32-bit words (three for BF16, six for F32); rows past the
// resource bound read 0.
template <typename T> struct PairRow {
  static constexpr int kWords = 3 * static_cast<int>(sizeof(T)) / 2;
  uint32_t word[kWords];
  __device__ void load(__amdgpu_buffer_rsrc_t resource, uint32_t lane, uint32_t row) {
#pragma unroll
    for (int i = 0; i < kWords; ++i)
      word[i] = __builtin_amdgcn_raw_buffer_load_b32(resource,
                                                     static_cast<int>(lane + row + 4 * i), 0, 0);
  }
  __device__ float at(int i) const {
    if constexpr (sizeof(T) == 2)
      return __builtin_bit_cast(float, (i & 1) != 0 ? word[i >> 1] & 0xffff0000U
                                                    : word[i >> 1] << 16);
    else
      return __builtin_bit_cast(float, word[i]);
  }
};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// {bf16(a), bf16(b)} in one v_cvt_pk_bf16_f32 (round to nearest even).
__device__ inline uint32_t pack_bf16(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// {fp16(a), fp16(b)}, round to nearest even, saturated to +-65504.
__device__ inline uint32_t pack_f16(float a, float b) {
  const f32x2 v = {fminf(fmaxf(a, -65504.0F), 65504.0F), fminf(fmaxf(b, -65504.0F), 65504.0F)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
// One 16-bit plane: BF16 (uint16_t *) or FP16 (F16Out).
template <typename O> struct Plane16;
template <> struct Plane16<uint16_t *> {
  static __device__ uint16_t *ptr(uint16_t *o) { return o; }
  static __device__ int *flag(uint16_t *) { return nullptr; }
  static __device__ uint32_t pack(float a, float b) { return pack_bf16(a, b); }
};
template <> struct Plane16<F16Out> {
  static __device__ uint16_t *ptr(const F16Out &o) { return o.out; }
  static __device__ int *flag(const F16Out &o) { return o.saturated; }
  static __device__ uint32_t pack(float a, float b) { return pack_f16(a, b); }
};
// Range check of FP16 outputs (no-op for BF16 planes, whose flag is null):
// one branch per pair or per eight values.
__device__ inline void note_pair(int *flag, float a, float b) {
  if (flag != nullptr && !(__builtin_fabsf(a) <= 65504.0F && __builtin_fabsf(b) <= 65504.0F))
    atomicOr(flag, kFlagF16Range);
}
__device__ inline void note_eight(int *flag, const float (&v)[8]) {
  if (flag == nullptr)
    return;
  bool out_of_range = false;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    out_of_range |= !(__builtin_fabsf(v[i]) <= 65504.0F);
  if (out_of_range)
    atomicOr(flag, kFlagF16Range);
}

// Output of a channel pair through segment-bounded buffer resources:
// `lane` is the pair's byte offset within a row of one plane, `row` the
// row's byte offset from the segment start.
template <typename O> struct PairOut;
template <> struct PairOut<float *> {
  __amdgpu_buffer_rsrc_t out;
  __device__ PairOut(float *o, size_t first, size_t rows, size_t W) {
    out = buffer_resource(o + first * W, static_cast<uint32_t>(rows * W * 4));
  }
  __device__ void put(uint32_t lane, uint32_t row, float a, float b) const {
    // The row offset goes into voffset: soffset is not part of the buffer
    // range check, so only voffset bounds the rows past the segment end.
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, a), out,
                                          static_cast<int>(2 * (lane + row)), 0, kStreamStore);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, b), out,
                                          static_cast<int>(2 * (lane + row) + 4), 0, kStreamStore);
  }
};
template <typename O> struct PairOut16 {
  __amdgpu_buffer_rsrc_t out;
  int *flag;
  __device__ PairOut16(const O &o, size_t first, size_t rows, size_t W) {
    out = buffer_resource(Plane16<O>::ptr(o) + first * W, static_cast<uint32_t>(rows * W * 2));
    flag = Plane16<O>::flag(o);
  }
  __device__ void put(uint32_t lane, uint32_t row, float a, float b) const {
    note_pair(flag, a, b);
    __builtin_amdgcn_raw_buffer_store_b32(Plane16<O>::pack(a, b), out,
                                          static_cast<int>(lane + row), 0, kStreamStore);
  }
};
template <> struct PairOut<uint16_t *> : PairOut16<uint16_t *> {
  using PairOut16<uint16_t *>::PairOut16;
};
template <> struct PairOut<F16Out> : PairOut16<F16Out> {
  using PairOut16<F16Out>::PairOut16;
};
template <> struct PairOut<SplitOut> {
  __amdgpu_buffer_rsrc_t hi, lo;
  bool has_lo;
  __device__ PairOut(const SplitOut &o, size_t first, size_t rows, size_t W) {
    hi = buffer_resource(o.hi + first * W, static_cast<uint32_t>(rows * W * 2));
    has_lo = o.lo != nullptr;
    lo = buffer_resource(has_lo ? o.lo + first * W : o.hi, has_lo ? static_cast<uint32_t>(rows * W * 2) : 0);
  }
  __device__ void put(uint32_t lane, uint32_t row, float a, float b) const {
    const uint32_t h = pack_bf16(a, b);
    __builtin_amdgcn_raw_buffer_store_b32(h, hi, static_cast<int>(lane + row), 0, kStreamStore);
    // With no lo plane the resource has zero size and the store is dropped.
    __builtin_amdgcn_raw_buffer_store_b32(
        pack_bf16(a - __builtin_bit_cast(float, h << 16),
                  b - __builtin_bit_cast(float, h & 0xffff0000U)),
        lo, static_cast<int>(lane + row), 0, kStreamStore);
  }
};

template <typename T, int kWin, int kTaps, bool kDirect>
struct PairFir {
  float stap[6][kWin], ftap[kTaps], d[2];
  float swin[6][kWin], uwin[2][kTaps];  // slot kWin-1 / kTaps-1 is the newest

  // One row: shifts the six projection values and u into the windows and
  // returns the pair's outputs y = x2 * (FIR(u) [+ d * u]).
  __device__ void step(const PairRow<T> &row, float (&y)[2]) {
    float fir[6];
#pragma unroll
    for (int col = 0; col < 6; ++col) {
#pragma unroll
      for (int i = 0; i < kWin - 1; ++i)
        swin[col][i] = swin[col][i + 1];
      swin[col][kWin - 1] = row.at(col);
      float total = 0.0F;
#pragma unroll
      for (int i = 0; i < kWin; ++i)
        total += swin[col][i] * stap[col][i];
      fir[col] = total;
    }
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      const float u = fir[3 * ch + 1] * fir[3 * ch + 2];
#pragma unroll
      for (int i = 0; i < kTaps - 1; ++i)
        uwin[ch][i] = uwin[ch][i + 1];
      uwin[ch][kTaps - 1] = u;
      float total = 0.0F;
#pragma unroll
      for (int i = 0; i < kTaps; ++i)
        total += uwin[ch][i] * ftap[i];
      if constexpr (kDirect)
        total += d[ch] * u;
      y[ch] = fir[3 * ch] * total;
    }
  }
};

template <typename T, typename O, int kWin, int kTaps, bool kDirect>
__global__ __launch_bounds__(kStreamWaves * 64) void hyena_fir_stream_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len,
    const float *__restrict__ inner_history, const float *__restrict__ filter,
    size_t group_size, int k, int causal, const float *__restrict__ direct,
    size_t L, size_t W, unsigned channel_blocks, unsigned segments, unsigned seg_len, O out) {
  constexpr int kLead = (kTaps - 1) + (kWin - 1);
  // XCD-aware order: consecutive hardware ids go to different XCDs, so each
  // XCD takes a contiguous band of segments (neighbouring segments share
  // their lead rows through that XCD's L2).
  const unsigned total = channel_blocks * segments;
  const unsigned xcd = blockIdx.x % 8, q = total / 8, r = total % 8;
  const unsigned linear = xcd * q + min(xcd, r) + blockIdx.x / 8;
  const unsigned segment = linear / channel_blocks;
  const unsigned cblock = linear % channel_blocks;
  const int lane = threadIdx.x & 63;
  const size_t c = cblock * static_cast<size_t>(kStreamChannels) +
                   (threadIdx.x >> 6) * 128 + 2 * lane;
  if (c >= W)
    return;
  const size_t t0 = static_cast<size_t>(segment) * seg_len;
  const uint32_t seg_rows = static_cast<uint32_t>(min(L - t0, static_cast<size_t>(seg_len)));
  const size_t cols3 = 3 * W;

  PairFir<T, kWin, kTaps, kDirect> fir;
#pragma unroll
  for (int ch = 0; ch < 2; ++ch) {
    float t3[3][kWin];
    load_window_taps(short_filter, short_len, c + ch, t3);
#pragma unroll
    for (int s = 0; s < 3; ++s)
#pragma unroll
      for (int i = 0; i < kWin; ++i)
        fir.stap[3 * ch + s][i] = t3[s][i];
  }
  const float *h = filter + (c / group_size) * k;
#pragma unroll
  for (int i = 0; i < kTaps; ++i) {
    const int j = i - (kTaps - k);
    fir.ftap[i] = j >= 0 ? h[causal ? k - 1 - j : j] : 0.0F;
  }
  if constexpr (kDirect) {
    fir.d[0] = direct[c];
    fir.d[1] = direct[c + 1];
  }

  const uint32_t row_bytes = static_cast<uint32_t>(cols3 * sizeof(T));
  const uint32_t lane_bytes = static_cast<uint32_t>(3 * c * sizeof(T));
  if (t0 >= static_cast<size_t>(kLead)) {
    // Interior segment: stream the lead rows through zeroed windows.
#pragma unroll
    for (int col = 0; col < 6; ++col)
#pragma unroll
      for (int i = 0; i < kWin; ++i)
        fir.swin[col][i] = 0.0F;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int i = 0; i < kTaps; ++i)
        fir.uwin[ch][i] = 0.0F;
    const auto lead = buffer_resource(P + (t0 - kLead) * cols3, kLead * row_bytes);
    PairRow<T> rows[kLead];
#pragma unroll
    for (int b = 0; b < kLead; ++b)
      rows[b].load(lead, lane_bytes, b * row_bytes);
#pragma unroll
    for (int b = 0; b < kLead; ++b) {
      float y[2];
      fir.step(rows[b], y);
    }
  } else {
    // First segment: the windows start from the caches (zeros without
    // them); slot i holds row i - kWin (short FIR) or i - kTaps (u).
#pragma unroll
    for (int col = 0; col < 6; ++col)
#pragma unroll
      for (int i = 0; i < kWin; ++i) {
        const long hrow = static_cast<long>(short_len - 1) + i - kWin;
        fir.swin[col][i] = (short_history != nullptr && hrow >= 0)
                               ? short_history[static_cast<size_t>(hrow) * cols3 + 3 * c + col]
                               : 0.0F;
      }
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int i = 0; i < kTaps; ++i) {
        const long hrow = static_cast<long>(k - 1) + i - kTaps;
        fir.uwin[ch][i] = (inner_history != nullptr && hrow >= 0)
                              ? inner_history[static_cast<size_t>(hrow) * W + c + ch]
                              : 0.0F;
      }
  }

  // Segment rows: loads past the sequence end read 0, stores past it drop.
  const auto in = buffer_resource(P + t0 * cols3, seg_rows * row_bytes);
  const PairOut<O> sink(out, t0, seg_rows, W);
  const uint32_t out_lane = static_cast<uint32_t>(c * 2);
  const uint32_t out_row = static_cast<uint32_t>(W * 2);
  PairRow<T> next[kStreamBatch];
#pragma unroll
  for (int b = 0; b < kStreamBatch; ++b)
    next[b].load(in, lane_bytes, b * row_bytes);
  for (uint32_t base = 0; base < seg_rows; base += kStreamBatch) {
    PairRow<T> cur[kStreamBatch];
#pragma unroll
    for (int b = 0; b < kStreamBatch; ++b)
      cur[b] = next[b];
    if (base + kStreamBatch < seg_rows) {
#pragma unroll
      for (int b = 0; b < kStreamBatch; ++b)
        next[b].load(in, lane_bytes, (base + kStreamBatch + b) * row_bytes);
    }
#pragma unroll
    for (int b = 0; b < kStreamBatch; ++b) {
      float y[2];
      fir.step(cur[b], y);
      sink.put(out_lane, (base + b) * out_row, y[0], y[1]);
    }
  }
}

// ---- HCS / HCM on MFMA: the grouped FIR of a 16-channel slice as a
// Toeplitz product. For output rows [r0, r0+16) and window rows
// i = r0 .. r0+159 (window row i holds u at t0 - (k-1) + i):
//
//   Y[r][c] = sum_i T[r][i - r0] * U[i][c],   T[r][j] = h[tap(j - r)]
//
// where old = j - r in [0, k) is the distance from the oldest row of the
// filter span (cross-correlation pairs it with tap `old`, causal convolution
// with tap k-1-old) and T is 0 elsewhere. T does not depend on r0, so each
// wave builds its A fragments once. U is staged in LDS as split BF16 planes
// (u = hi + lo, |lo| <= 2^-9 |u|), transposed to [channel][row] so that one
// ds_read_b128 yields a B fragment; the taps are split the same way and
// three passes (h_hi u_hi + h_hi u_lo + h_lo u_hi) keep F32 accuracy. Every
// channel of a 16-column slice must share one filter group.
constexpr int kFirTile = 128;    // output rows per block
constexpr int kFirThreads = 1024; // 16 waves

template <int kMaxTaps>
struct FirMfmaShape {
  static constexpr int kSteps = (16 + kMaxTaps - 1 + 31) / 32;  // K=32 steps per row block
  static constexpr int kSpan = (kFirTile - 16) + 32 * kSteps;   // window rows a read may touch
  // Row stride (BF16) of a channel: a multiple of 8 (16-byte reads) with an
  // odd number of 16-byte units, so 8 lanes on 8 channels hit 8 bank groups.
  static constexpr int kStride = ((kSpan + 7) / 8 % 2 == 1) ? (kSpan + 7) / 8 * 8
                                                             : (kSpan + 7) / 8 * 8 + 8;
  static constexpr size_t kLdsBytes =
      2 * kChannels * kStride * sizeof(uint16_t) + kFirTile * kChannels * sizeof(float);
};

// Toeplitz A fragments of every filter group: entry ((g * kSteps + q) * 2 +
// plane) * 64 + lane holds lane's 8 BF16 values of K step q (plane 0 = hi,
// 1 = lo of the F32 tap).
template <int kMaxTaps>
__global__ __launch_bounds__(64) void toeplitz_fragments_kernel(const float *__restrict__ filter,
                                                              int k, int causal,
                                                              uint4 *__restrict__ table) {
  constexpr int kSteps = FirMfmaShape<kMaxTaps>::kSteps;
  const int lane = threadIdx.x;
  const int q = blockIdx.y;
  const size_t g = blockIdx.x;
  const float *h = filter + g * k;
  uint16_t hi[8], lo[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int old = 32 * q + 8 * (lane >> 4) + e - (lane & 15);
    float tap = 0.0F;
    if (old >= 0 && old < k)
      tap = h[causal ? k - 1 - old : old];
    hi[e] = f32_to_bf16(tap);
    lo[e] = f32_to_bf16(tap - bf16_to_f32(hi[e]));
  }
  const size_t base = ((g * kSteps + q) * 2) * 64 + lane;
  table[base] = __builtin_bit_cast(uint4, hi);
  table[base + 64] = __builtin_bit_cast(uint4, lo);
}

__device__ inline bf16x8 load_frag(const uint16_t *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(p));
}

template <typename T, typename O, int kMaxTaps, int kWin>
__global__ __launch_bounds__(kFirThreads) void hyena_fir_mfma_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len,
    const float *__restrict__ inner_history, const uint4 *__restrict__ fragments,
    size_t group_size, int k, int causal, const float *__restrict__ direct,
    size_t L, size_t W, size_t planar, O out) {
  using Shape = FirMfmaShape<kMaxTaps>;
  extern __shared__ __attribute__((aligned(16))) unsigned char fir_smem[];
  uint16_t *u_hi = reinterpret_cast<uint16_t *>(fir_smem);    // [64][kStride]
  uint16_t *u_lo = u_hi + kChannels * Shape::kStride;         // [64][kStride]
  float *x2_s = reinterpret_cast<float *>(u_lo + kChannels * Shape::kStride);  // [kFirTile][64]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const size_t c_block = blockIdx.x * static_cast<size_t>(kChannels);
  const size_t c = c_block + lane;
  const long t0 = static_cast<long>(blockIdx.y) * kFirTile;
  const int hist = k - 1;
  const long window = kFirTile + hist;  // staged rows
  const size_t cols3 = 3 * W;

  // ---- Stage u (and x2 of the output rows): wave w owns a contiguous run
  // of kRows (even) window rows. Interior runs load all their rows (plus the
  // short-FIR lead-in) in one batch and evaluate the FIR from registers;
  // runs that touch the history, the window end or the sequence end take
  // the general path.
  {
    constexpr int kWaves = kFirThreads / 64;
    constexpr int kRows = ((Shape::kSpan + kWaves - 1) / kWaves + 1) / 2 * 2;
    const int i0 = wave * kRows, i1 = min(i0 + kRows, Shape::kSpan);
    const long tw = t0 - hist + i0;  // time of the run's first row
    const bool interior = tw - (kWin - 1) >= 0 && i0 + kRows <= window &&
                          tw + kRows <= static_cast<long>(L);
    if (interior) {
      float taps[3][kWin];
      load_window_taps(short_filter, short_len, c, taps);
      // Wave-uniform row pointers plus a 32-bit per-lane column offset
      // (scalar-base addressing, no per-lane 64-bit address arithmetic).
      const T *base = P + static_cast<size_t>(tw - (kWin - 1)) * cols3;
      const uint32_t row_bytes = static_cast<uint32_t>(cols3 * sizeof(T));
      const auto resource = buffer_resource(base, (kRows + kWin - 1) * row_bytes);
      uint32_t column[3];
#pragma unroll
      for (int s = 0; s < 3; ++s)
        column[s] = static_cast<uint32_t>(pcol(c, s, planar) * sizeof(T));
      float v[kRows + kWin - 1][3];
#pragma unroll
      for (int b = 0; b < kRows + kWin - 1; ++b)
#pragma unroll
        for (int s = 0; s < 3; ++s)
          v[b][s] = buffer_act<T>(resource, column[s], b * row_bytes);
      uint32_t *hi_pairs = reinterpret_cast<uint32_t *>(u_hi + lane * Shape::kStride + i0);
      uint32_t *lo_pairs = reinterpret_cast<uint32_t *>(u_lo + lane * Shape::kStride + i0);
#pragma unroll
      for (int b = 0; b < kRows; b += 2) {
        uint32_t hi_pair = 0, lo_pair = 0;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          float fir[3];
#pragma unroll
          for (int s = 0; s < 3; ++s) {
            float total = 0.0F;
#pragma unroll
            for (int j = 0; j < kWin; ++j)
              total += v[b + half + j][s] * taps[s][j];
            fir[s] = total;
          }
          const float u = fir[1] * fir[2];
          const uint16_t hi = f32_to_bf16(u);
          hi_pair |= static_cast<uint32_t>(hi) << (16 * half);
          lo_pair |= static_cast<uint32_t>(f32_to_bf16(u - bf16_to_f32(hi))) << (16 * half);
          if (i0 + b + half >= hist)
            x2_s[(i0 + b + half - hist) * kChannels + lane] = fir[0];
        }
        hi_pairs[b / 2] = hi_pair;
        lo_pairs[b / 2] = lo_pair;
      }
    } else {
      // Rows before t = 0 come from the inner history; rows past the window
      // or the sequence are zero (they only meet zero taps or unstored
      // outputs).
      int i = i0;
      for (; i < i1; ++i) {
        const long t = t0 - hist + i;
        if (t >= 0 && i < window && t < static_cast<long>(L))
          break;
        float u = 0.0F;
        if (t < 0 && i < window && inner_history != nullptr)
          u = inner_history[static_cast<size_t>(hist + t) * W + c];
        const uint16_t hi = f32_to_bf16(u);
        u_hi[lane * Shape::kStride + i] = hi;
        u_lo[lane * Shape::kStride + i] = f32_to_bf16(u - bf16_to_f32(hi));
      }
      const int i_end = static_cast<int>(min<long>(
          i1, min<long>(window, static_cast<long>(L) - (t0 - hist))));
      if (i < i_end) {
        RowStream<T, kWin> stream;
        load_window_taps(short_filter, short_len, c, stream.taps);
        stream.prime(P, short_history, short_len, cols3, planar, t0 - hist + i, c);
        for (; i < i_end; i += kBatch) {
          const size_t t = static_cast<size_t>(t0 - hist + i);
          float rows[kBatch][3];
          load_batch(P, cols3, planar, t, t + min(kBatch, i_end - i), c, rows);
#pragma unroll
          for (int b = 0; b < kBatch; ++b) {
            if (i + b >= i_end)
              break;
            float fir[3];
            stream.push(rows[b], fir);
            const float u = fir[1] * fir[2];
            const uint16_t hi = f32_to_bf16(u);
            u_hi[lane * Shape::kStride + i + b] = hi;
            u_lo[lane * Shape::kStride + i + b] = f32_to_bf16(u - bf16_to_f32(hi));
            if (i + b >= hist)
              x2_s[(i + b - hist) * kChannels + lane] = fir[0];
          }
        }
        i = i_end;
      }
      for (; i < i1; ++i) {
        u_hi[lane * Shape::kStride + i] = 0;
        u_lo[lane * Shape::kStride + i] = 0;
      }
    }
  }
  __syncthreads();

  // ---- Products: wave w takes channel slice w % 4 and row blocks w/4, +2, ...
  const int slice = wave & 3;
  const int ch = slice * 16 + (lane & 15);
  const size_t group = (c_block + slice * 16) / group_size;
  bf16x8 t_hi[Shape::kSteps], t_lo[Shape::kSteps];
#pragma unroll
  for (int q = 0; q < Shape::kSteps; ++q) {
    const size_t base = ((group * Shape::kSteps + q) * 2) * 64 + lane;
    t_hi[q] = __builtin_bit_cast(bf16x8, fragments[base]);
    t_lo[q] = __builtin_bit_cast(bf16x8, fragments[base + 64]);
  }
  const float d = direct != nullptr ? direct[c_block + ch] : 0.0F;
  const uint16_t *row_hi = u_hi + ch * Shape::kStride;
  const uint16_t *row_lo = u_lo + ch * Shape::kStride;
  for (int rb = wave >> 2; rb < kFirTile / 16; rb += kFirThreads / 64 / 4) {
    const int r0 = rb * 16;
    if (t0 + r0 >= static_cast<long>(L))
      break;
    f32x4 acc = {0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
    for (int q = 0; q < Shape::kSteps; ++q) {
      const int i = r0 + 32 * q + 8 * (lane >> 4);
      const bf16x8 b_hi = load_frag(row_hi + i);
      const bf16x8 b_lo = load_frag(row_lo + i);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(t_hi[q], b_hi, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(t_hi[q], b_lo, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(t_lo[q], b_hi, acc, 0, 0, 0);
    }
    // y replaces x2 in LDS (each element is read and written by one lane).
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = r0 + 4 * (lane >> 4) + e;
      float total = acc[e];
      if (direct != nullptr)
        total += d * (bf16_to_f32(row_hi[r + hist]) + bf16_to_f32(row_lo[r + hist]));
      x2_s[r * kChannels + ch] *= total;
    }
  }
  __syncthreads();
  // Row-contiguous stores: wave w writes rows w, w+16, ... across 64 channels.
  for (int r = wave; r < kFirTile; r += kFirThreads / 64) {
    const long t = t0 + r;
    if (t >= static_cast<long>(L))
      break;
    put_nt(out, static_cast<size_t>(t) * W + c, x2_s[r * kChannels + lane]);
  }
}

// ---- HCL on channel pairs (interleaved projection, short FIR of 3): the
// chunked scan of the modal recurrence with the row stream of the HCS kernel
// (12/24-byte loads of two channels per lane, packed non-temporal stores).
// A wave covers 128 channels of one kChunk-row chunk.
__device__ inline float swap_pair(float v) {
  // quad_perm [1, 0, 3, 2]: each lane reads its neighbour's value.
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}

template <typename T>
struct PairShort {
  // Lane half h computes the short FIR of its own channel c + h only; the
  // pair exchanges what the other lane needs through DPP swaps.
  float stap[3][3], swin[3][3];  // slot 2 is the newest row
  uint32_t sel[3];                // BF16 rows: byte selectors of the own columns
  int half;
  __device__ void taps(const uint16_t *short_filter, size_t c) {
    half = threadIdx.x & 1;
    load_window_taps(short_filter, 3, c + half, stap);
    // The pair's row words are [c col0 | c col1], [c col2 | c+1 col0],
    // [c+1 col1 | c+1 col2]; v_perm moves the own column's two bytes into
    // the high half (low half zero), which is its F32 value.
    sel[0] = half ? 0x07060c0cU : 0x01000c0cU;  // perm(w1, w0)
    sel[1] = half ? 0x05040c0cU : 0x03020c0cU;  // perm(w2, w0)
    sel[2] = half ? 0x07060c0cU : 0x01000c0cU;  // perm(w2, w1)
  }
  // Window before row t0: rows t0-2, t0-1 from P, or from the short history
  // (F32 [2][3W]) when they precede row 0.
  __device__ void prime(const T *P, const float *short_history, size_t t0, size_t W, size_t c) {
    const size_t cols3 = 3 * W;
    const size_t own = 3 * (c + half);
#pragma unroll
    for (int i = 1; i < 3; ++i) {
      const long row = static_cast<long>(t0) - 3 + i;
#pragma unroll
      for (int col = 0; col < 3; ++col) {
        float v = 0.0F;
        if (row >= 0)
          v = load_act(P, static_cast<size_t>(row) * cols3 + own + col);
        else if (short_history != nullptr && row + 2 >= 0)
          v = short_history[static_cast<size_t>(row + 2) * cols3 + own + col];
        swin[col][i] = v;
      }
    }
  }
  // Shifts in one row; x2 and u of the own channel, u of the other.
  __device__ void step(const PairRow<T> &row, float &x2, float &u_own, float &u_other) {
    float v[3];
    if constexpr (sizeof(T) == 2) {
      v[0] = __builtin_bit_cast(float, __builtin_amdgcn_perm(row.word[1], row.word[0], sel[0]));
      v[1] = __builtin_bit_cast(float, __builtin_amdgcn_perm(row.word[2], row.word[0], sel[1]));
      v[2] = __builtin_bit_cast(float, __builtin_amdgcn_perm(row.word[2], row.word[1], sel[2]));
    } else {
#pragma unroll
      for (int col = 0; col < 3; ++col)
        v[col] = __builtin_bit_cast(float, half ? row.word[3 + col] : row.word[col]);
    }
    float fir[3];
#pragma unroll
    for (int col = 0; col < 3; ++col) {
      swin[col][0] = swin[col][1];
      swin[col][1] = swin[col][2];
      swin[col][2] = v[col];
      float total = 0.0F;
#pragma unroll
      for (int i = 0; i < 3; ++i)
        total += swin[col][i] * stap[col][i];
      fir[col] = total;
    }
    x2 = fir[0];
    u_own = fir[1] * fir[2];
    u_other = swap_pair(u_own);
  }
};

constexpr int kHclBatch = 4;  // even: the output pass stores rows in pairs

// Lanes l and l ^ 1 share a channel pair: lane half h = l & 1 runs the short
// FIR of channel c + h ("own"; the partner's is "other") and keeps modal
// states 8h .. 8h+7 of both channels. Per row the pair swaps u, the partial
// modal sums of the partner's channel and y (DPP), so each lane computes y
// of its own channel only. Arrays indexed [0] own, [1] other.
constexpr int kHclHalf = kMaxState / 2;


// Phase 1: final local state of every chunk from a zero start.
template <typename T>
__global__ __launch_bounds__(256) void hcl_state_pair_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, size_t L, size_t W,
    const float *__restrict__ poles, int S, float *__restrict__ chunk_state) {
  const int lane = threadIdx.x & 63, half = lane & 1;
  const size_t c = blockIdx.x * 256ULL + (threadIdx.x >> 6) * 64 + 2 * (lane >> 1);
  if (c >= W)
    return;
  const size_t g = blockIdx.y;
  const size_t t0 = g * kChunk;
  const uint32_t rows = static_cast<uint32_t>(min(L - t0, static_cast<size_t>(kChunk)));
  PairShort<T> sh;
  sh.taps(short_filter, c);
  sh.prime(P, short_history, t0, W, c);
  float p[2][kHclHalf], st[2][kHclHalf];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch)
#pragma unroll
    for (int i = 0; i < kHclHalf; ++i) {
      const int m = kHclHalf * half + i;
      p[ch][i] = m < S ? poles[(c + (ch ^ half)) * S + m] : 0.0F;
      st[ch][i] = 0.0F;
    }
  const uint32_t row_bytes = static_cast<uint32_t>(3 * W * sizeof(T));
  const auto in = buffer_resource(P + t0 * 3 * W, rows * row_bytes);
  const uint32_t lane_bytes = static_cast<uint32_t>(3 * c * sizeof(T));
  PairRow<T> next[kHclBatch];
#pragma unroll
  for (int b = 0; b < kHclBatch; ++b)
    next[b].load(in, lane_bytes, b * row_bytes);
  for (uint32_t base = 0; base < rows; base += kHclBatch) {
    PairRow<T> cur[kHclBatch];
#pragma unroll
    for (int b = 0; b < kHclBatch; ++b)
      cur[b] = next[b];
    if (base + kHclBatch < rows) {
#pragma unroll
      for (int b = 0; b < kHclBatch; ++b)
        next[b].load(in, lane_bytes, (base + kHclBatch + b) * row_bytes);
    }
#pragma unroll
    for (int b = 0; b < kHclBatch; ++b) {
      if (base + b >= rows)
        break;
      float x2, u[2];
      sh.step(cur[b], x2, u[0], u[1]);
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int i = 0; i < kHclHalf; ++i)
          st[ch][i] = p[ch][i] * st[ch][i] + u[ch];
    }
  }
#pragma unroll
  for (int i = 0; i < kHclHalf; ++i) {
    const int m = kHclHalf * half + i;
    if (m < S)
      *reinterpret_cast<float2 *>(&chunk_state[(g * S + m) * W + c]) =
          half == 0 ? make_float2(st[0][i], st[1][i]) : make_float2(st[1][i], st[0][i]);
  }
}

// Phase 2: chunk-start states in place (and the final state), four segments
// of chunks per (state, channel) in one block: each segment folds its chunks,
// the segments combine through LDS, each segment rescans its chunks.
__global__ __launch_bounds__(256) void hcl_carry_seg_kernel(
    float *__restrict__ chunk_state, size_t G, size_t L, size_t W, int S,
    const float *__restrict__ poles, float *__restrict__ modal_state) {
  __shared__ float fold[4][64], power_s[4][64];
  const int lane = threadIdx.x & 63, seg = threadIdx.x >> 6;
  const size_t c = blockIdx.x * 64ULL + lane;
  const int m = static_cast<int>(blockIdx.y);
  const bool valid = c < W;
  const float p = valid ? poles[c * S + m] : 0.0F;
  float full = p;  // p^kChunk by repeated squaring (kChunk is a power of two)
  for (int e = 1; e < kChunk; e <<= 1)
    full *= full;
  const size_t per = (G + 3) / 4;
  const size_t g0 = min(G, seg * per), g1 = min(G, g0 + per);
  auto chunk_power = [&](size_t g) {
    const size_t len = min(L - g * kChunk, static_cast<size_t>(kChunk));
    if (len == static_cast<size_t>(kChunk))
      return full;
    float power = 1.0F;
    for (size_t e = 0; e < len; ++e)
      power *= p;
    return power;
  };
  // Fold: the segment's state from a zero start and its total power.
  float state = 0.0F, power = 1.0F;
  if (valid)
    for (size_t g = g0; g < g1; ++g) {
      const float pw = chunk_power(g);
      state = pw * state + chunk_state[(g * S + m) * W + c];
      power *= pw;
    }
  fold[seg][lane] = state;
  power_s[seg][lane] = power;
  __syncthreads();
  float in = (valid && modal_state != nullptr) ? modal_state[c * S + m] : 0.0F;
  for (int q = 0; q < seg; ++q)
    in = power_s[q][lane] * in + fold[q][lane];
  if (!valid)
    return;
  // Rescan: chunk g's start state, written in place of its local state.
  state = in;
  for (size_t g = g0; g < g1; ++g) {
    const float local = chunk_state[(g * S + m) * W + c];
    chunk_state[(g * S + m) * W + c] = state;
    state = chunk_power(g) * state + local;
  }
  if (seg == 3 && modal_state != nullptr)
    modal_state[c * S + m] = state;
}

// Phase 3: rescan every chunk from its true start state and write y. Both
// lanes of a pair hold y of both channels. Rows leave in pairs: for BF16 and
// split outputs the even lane writes the first row's word (both channels;
// hi and lo planes through two uniform resources), the odd lane the second
// row's; for F32 each lane writes its own channel of both rows.
template <typename O> struct HalfOut;
template <> struct HalfOut<float *> {
  __amdgpu_buffer_rsrc_t out;
  __device__ HalfOut(float *o, size_t first, size_t rows, size_t W) {
    out = buffer_resource(o + first * W, static_cast<uint32_t>(rows * W * 4));
  }
  __device__ void put(int half, uint32_t lane, uint32_t row, float a, float b) const {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, half ? b : a), out,
                                          static_cast<int>(2 * (lane + row) + 4 * half), 0,
                                          kStreamStore);
  }
  __device__ void put_rows(int half, uint32_t lane, uint32_t row, uint32_t row_bytes, float a0,
                           float b0, float a1, float b1) const {
    put(half, lane, row, a0, b0);
    put(half, lane, row + row_bytes, a1, b1);
  }
};
template <typename O> struct HalfOut16 {
  __amdgpu_buffer_rsrc_t out;
  int *flag;
  __device__ HalfOut16(const O &o, size_t first, size_t rows, size_t W) {
    out = buffer_resource(Plane16<O>::ptr(o) + first * W, static_cast<uint32_t>(rows * W * 2));
    flag = Plane16<O>::flag(o);
  }
  __device__ void put_rows(int half, uint32_t lane, uint32_t row, uint32_t row_bytes, float a0,
                           float b0, float a1, float b1) const {
    // Even lane row `row`, odd lane the next one.
    if (half == 0)
      note_pair(flag, a0, b0);
    else
      note_pair(flag, a1, b1);
    const uint32_t word = half == 0 ? Plane16<O>::pack(a0, b0) : Plane16<O>::pack(a1, b1);
    __builtin_amdgcn_raw_buffer_store_b32(word, out,
                                          static_cast<int>(lane + row + half * row_bytes), 0,
                                          kStreamStore);
  }
};
template <> struct HalfOut<uint16_t *> : HalfOut16<uint16_t *> {
  using HalfOut16<uint16_t *>::HalfOut16;
};
template <> struct HalfOut<F16Out> : HalfOut16<F16Out> {
  using HalfOut16<F16Out>::HalfOut16;
};
template <> struct HalfOut<SplitOut> {
  // Both resources are uniform; a missing lo plane gets an empty one (its
  // stores are dropped).
  __amdgpu_buffer_rsrc_t hi, lo;
  __device__ HalfOut(const SplitOut &o, size_t first, size_t rows, size_t W) {
    const uint32_t bytes = static_cast<uint32_t>(rows * W * 2);
    hi = buffer_resource(o.hi + first * W, bytes);
    lo = buffer_resource(o.lo != nullptr ? o.lo + first * W : o.hi, o.lo != nullptr ? bytes : 0);
  }
  // Two rows of the pair's channels (a: channel c, b: channel c + 1): the even
  // lane writes row `row`, the odd lane the next one, each both planes.
  __device__ void put_rows(int half, uint32_t lane, uint32_t row, uint32_t row_bytes, float a0,
                           float b0, float a1, float b1) const {
    const float a = half == 0 ? a0 : a1, b = half == 0 ? b0 : b1;
    const uint32_t h = pack_bf16(a, b);
    const uint32_t l = pack_bf16(a - __builtin_bit_cast(float, h << 16),
                                 b - __builtin_bit_cast(float, h & 0xffff0000U));
    const int offset = static_cast<int>(lane + row + half * row_bytes);
    __builtin_amdgcn_raw_buffer_store_b32(h, hi, offset, 0, kStreamStore);
    __builtin_amdgcn_raw_buffer_store_b32(l, lo, offset, 0, kStreamStore);
  }
};

template <typename T, typename O>
__global__ __launch_bounds__(256) void hcl_output_pair_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, size_t L, size_t W,
    const float *__restrict__ poles, const float *__restrict__ residues,
    const float *__restrict__ direct, int S, const float *__restrict__ chunk_state, O out) {
  const int lane = threadIdx.x & 63, half = lane & 1;
  const size_t c = blockIdx.x * 256ULL + (threadIdx.x >> 6) * 64 + 2 * (lane >> 1);
  if (c >= W)
    return;
  const size_t g = blockIdx.y;
  const size_t t0 = g * kChunk;
  const uint32_t rows = static_cast<uint32_t>(min(L - t0, static_cast<size_t>(kChunk)));
  PairShort<T> sh;
  sh.taps(short_filter, c);
  sh.prime(P, short_history, t0, W, c);
  float p[2][kHclHalf], r[2][kHclHalf], st[2][kHclHalf], d[2];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch) {
    const size_t cc = c + (ch ^ half);
#pragma unroll
    for (int i = 0; i < kHclHalf; ++i) {
      const int m = kHclHalf * half + i;
      p[ch][i] = m < S ? poles[cc * S + m] : 0.0F;
      r[ch][i] = m < S ? residues[cc * S + m] : 0.0F;
      st[ch][i] = m < S ? chunk_state[(g * S + m) * W + cc] : 0.0F;
    }
    d[ch] = direct[cc];
  }
  const uint32_t row_bytes = static_cast<uint32_t>(3 * W * sizeof(T));
  const auto in = buffer_resource(P + t0 * 3 * W, rows * row_bytes);
  const uint32_t lane_bytes = static_cast<uint32_t>(3 * c * sizeof(T));
  const HalfOut<O> sink(out, t0, rows, W);
  const uint32_t out_lane = static_cast<uint32_t>(c * 2);
  const uint32_t out_row = static_cast<uint32_t>(W * 2);
  PairRow<T> next[kHclBatch];
#pragma unroll
  for (int b = 0; b < kHclBatch; ++b)
    next[b].load(in, lane_bytes, b * row_bytes);
  for (uint32_t base = 0; base < rows; base += kHclBatch) {
    PairRow<T> cur[kHclBatch];
#pragma unroll
    for (int b = 0; b < kHclBatch; ++b)
      cur[b] = next[b];
    if (base + kHclBatch < rows) {
#pragma unroll
      for (int b = 0; b < kHclBatch; ++b)
        next[b].load(in, lane_bytes, (base + kHclBatch + b) * row_bytes);
    }
    float ya[2], yb[2];  // channels c and c + 1 of the batch's last two rows
#pragma unroll
    for (int b = 0; b < kHclBatch; ++b) {
      float x2, u[2], modal[2];
      sh.step(cur[b], x2, u[0], u[1]);
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        modal[ch] = 0.0F;
#pragma unroll
        for (int i = 0; i < kHclHalf; ++i) {
          st[ch][i] = p[ch][i] * st[ch][i] + u[ch];
          modal[ch] += r[ch][i] * st[ch][i];
        }
      }
      // The partner's partial sum of the own channel; states 0..7 first,
      // then 8..15.
      const float partner = swap_pair(modal[1]);
      const float total = half == 0 ? modal[0] + partner : partner + modal[0];
      const float y = x2 * (total + d[0] * u[0]);
      const float y_other = swap_pair(y);
      ya[b & 1] = half == 0 ? y : y_other;
      yb[b & 1] = half == 0 ? y_other : y;
      // Rows past the chunk end are dropped by the store bound.
      if (b & 1)
        sink.put_rows(half, out_lane, (base + b - 1) * out_row, out_row, ya[0], yb[0], ya[1],
                      yb[1]);
    }
  }
}

// ---- Grouped FIR with k <= 128 (HCM) as a row stream on MFMA.
// A block owns 64 channels (four 16-channel slices, one per wave; each slice
// lies in one filter group) and a segment of kMsSegment output rows (fewer,
// down to kMsMinSegment, while the grid would have under kMsMinBlocks
// blocks: a 1024-token prompt at W = 4096 gets 256 blocks, not 64), walked
// in steps of 32 rows:
//  1. production (all lanes, two adjacent channels x 4 rows each): short FIR
//     and gates from the projection rows, u as split BF16 planes into LDS
//     ([channel][row], so one ds_read_b128 is a B fragment) and x2 into LDS;
//  2. each wave appends the new 32-row B fragments to a register ring of the
//     last five steps (the 160-row window that output rows r0..r0+31 read)
//     and forms Y = T . U on v_mfma_f32_16x16x32_bf16 for both 16-row
//     halves. The taps are BF16 values (as stored in evo2 artifacts), so the
//     product is exact in two passes, T U_hi + T U_lo; the Toeplitz A
//     fragments T_h[q] depend only on the filter group, so each lane builds
//     its 80 tap values once. Short FIR length 3 (the Evo 2 value);
//  3. the epilogue y = x2 * (Y + d u) goes through LDS and leaves as whole
//     rows of 64 channels (non-temporal stores bounded to the segment).
// A segment after the first starts kMsLead steps (128 rows) early to fill
// the ring; the first segment fills it from the inner history instead.
constexpr int kMsStep = 32;
constexpr int kMsK = 5;             // K steps in the window
constexpr int kMsChannels = 64;
constexpr int kMsSegment = 1024;
constexpr int kMsMinSegment = 256;
constexpr unsigned kMsMinBlocks = 256;
constexpr int kMsLead = 4;
constexpr int kMsUStride = 40;      // BF16 per channel in the u stage (80 B)

// Column of row `row` (0..31) of channel c in the u stage: 8-row units
// XOR-swizzled by (c >> 3) & 3, so the production writes of 16 lanes (16
// even channels, one unit) and the fragment reads of 8 lanes (8 consecutive
// channels) hit distinct banks; 8-row units stay 16-byte aligned.
__device__ inline int ms_ucol(int c, int row) {
  return (((row >> 3) ^ ((c >> 3) & 3)) << 3) + (row & 7);
}

template <typename O> struct MsOut;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
// One 16-byte non-temporal store (global_store_dwordx4 nt).
__device__ inline void store16_nt(void *dst, const void *lds_src) {
  __builtin_nontemporal_store(*reinterpret_cast<const u32x4 *>(lds_src),
                              reinterpret_cast<u32x4 *>(dst));
}
// y is staged in LDS as F32 [row][64]; the flush writes whole rows: lane ->
// row tid / 8, channels (tid % 8) * 8 .. + 7, converting to the output type
// there. `index` is the lane's first output element; the caller skips rows
// at or past the segment end. `stores` is the number of store instructions a
// wave issues per flush.
// (No __builtin_bit_cast of a vector element anywhere in this file: this
// compiler folds such a cast to element 0.)
__device__ inline void load8(const float *s, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4 *>(s);
  const f32x4 b = *reinterpret_cast<const f32x4 *>(s + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = a[i];
    v[4 + i] = b[i];
  }
}
__device__ inline void store16_words(void *dst, const uint32_t (&w)[4]) {
  const u32x4 v = {w[0], w[1], w[2], w[3]};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(dst));
}
template <> struct MsOut<float *> {
  __device__ static void flush(const float *src, float *out, size_t index) {
    store16_nt(out + index, src);
    store16_nt(out + index + 4, src + 4);
  }
};
template <typename O> struct MsOut16 {
  __device__ static void flush(const float *src, const O &out, size_t index) {
    float v[8];
    load8(src, v);
    note_eight(Plane16<O>::flag(out), v);
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = Plane16<O>::pack(v[2 * i], v[2 * i + 1]);
    store16_words(Plane16<O>::ptr(out) + index, w);
  }
};
template <> struct MsOut<uint16_t *> : MsOut16<uint16_t *> {};
template <> struct MsOut<F16Out> : MsOut16<F16Out> {};
template <> struct MsOut<SplitOut> {
  __device__ static void flush(const float *src, const SplitOut &out, size_t index) {
    float v[8];
    load8(src, v);
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hi[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
      lo[i] = pack_bf16(v[2 * i] - __builtin_bit_cast(float, hi[i] << 16),
                        v[2 * i + 1] - __builtin_bit_cast(float, hi[i] & 0xffff0000U));
    }
    store16_words(out.hi + index, hi);
    if (out.lo != nullptr)
      store16_words(out.lo + index, lo);
  }
};

// Two blocks per CU for BF16 projections (71 KB of LDS); F32 projection
// rows double the DMA stage (97 KB), so one block per CU.
template <typename T, typename O>
__global__ __launch_bounds__(256, sizeof(T) == 2 ? 2 : 1) void hyena_fir_mfma_stream_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len,
    const float *__restrict__ inner_history, const float *__restrict__ filter,
    size_t group_size, int k, int causal, const float *__restrict__ direct,
    size_t L, size_t W, unsigned channel_blocks, unsigned segments, unsigned seg_len, O out) {
  constexpr int kWin = 3;          // short FIR length
  constexpr int kRows = kWin + 3;  // projection rows per production lane
  // Projection stage of one step: rows R0 - 2 .. R0 + 31 of the block's 64
  // channels (384 B per row in BF16), copied by DMA kMsStages - 1 steps ahead.
  constexpr int kStageRows = kMsStep + kWin - 1;
  constexpr int kRowBytes = kMsChannels * 3 * static_cast<int>(sizeof(T));
  constexpr int kUnits = kStageRows * kRowBytes / 16;      // 16-byte DMA units
  constexpr int kUnitsPerRow = kRowBytes / 16;
  constexpr int kDmaPerStep = (kUnits + 255) / 256;        // per thread
  constexpr int kDmaMin = kUnits / 256;                    // per wave, at least
  constexpr int kStages = 2;
  // Software pipeline: in phase s the block flushes step s-1, produces step
  // s+1 and multiplies step s, so u is double buffered and x2 (overwritten in
  // place by y) triple buffered.
  __shared__ __attribute__((aligned(16))) unsigned char p_s[kStages][kStageRows * kRowBytes];
  __shared__ __attribute__((aligned(16))) uint16_t u_s[2][2][kMsChannels][kMsUStride];
  __shared__ __attribute__((aligned(16))) float xy_s[3][kMsStep][kMsChannels];

  const unsigned total = channel_blocks * segments;
  const unsigned xcd = blockIdx.x % 8, q8 = total / 8, r8 = total % 8;
  const unsigned linear = xcd * q8 + min(xcd, r8) + blockIdx.x / 8;
  const unsigned segment = linear / channel_blocks;
  const size_t c0 = static_cast<size_t>(linear % channel_blocks) * kMsChannels;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const size_t t0 = static_cast<size_t>(segment) * seg_len;
  const uint32_t seg_rows = static_cast<uint32_t>(min(L - t0, static_cast<size_t>(seg_len)));
  const int lead = t0 == 0 ? 0 : kMsLead;
  const size_t t_start = t0 - static_cast<size_t>(lead) * kMsStep;  // first produced row
  const int steps = lead + static_cast<int>((seg_rows + kMsStep - 1) / kMsStep);
  const size_t cols3 = 3 * W;

  // ---- Production lane: channels cp, cp + 1 and rows 4 * rg .. + 3 of a step.
  const int pair = tid & 31, rg = tid >> 5;
  const size_t cp = c0 + 2 * pair;
  float stap[6][kWin];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch) {
    float t3[3][kWin];
    load_window_taps(short_filter, short_len, cp + ch, t3);
#pragma unroll
    for (int s = 0; s < 3; ++s)
#pragma unroll
      for (int i = 0; i < kWin; ++i)
        stap[3 * ch + s][i] = t3[s][i];
  }
  // DMA of step `step` into stage `step % kStages`: rows clamp to [0, L), so
  // no access leaves the tensor (rows before 0 are replaced from the short
  // history in production; rows past L only feed outputs that are dropped).
  // Per-lane unit offsets within a stage (row within the stage, 16-byte
  // part within the row), fixed for the whole walk.
  uint32_t unit_row[kDmaPerStep], unit_byte[kDmaPerStep];
#pragma unroll
  for (int j = 0; j < kDmaPerStep; ++j) {
    const int unit = min(j * 256 + tid, kUnits - 1);
    unit_row[j] = static_cast<uint32_t>(unit / kUnitsPerRow);
    unit_byte[j] = static_cast<uint32_t>(unit_row[j] * cols3 * sizeof(T) +
                                         16 * (unit % kUnitsPerRow));
  }
  const unsigned char *p_block = reinterpret_cast<const unsigned char *>(P + 3 * c0);
  auto issue = [&](int step) {
    const long r_first = static_cast<long>(t_start) + step * kMsStep - (kWin - 1);
    unsigned char *stage = p_s[step % kStages];
    const bool inside = r_first >= 0 && r_first + kStageRows <= static_cast<long>(L);
    const unsigned char *base = p_block + static_cast<size_t>(max(r_first, 0L)) * cols3 * sizeof(T);
#pragma unroll
    for (int j = 0; j < kDmaPerStep; ++j) {
      if (j * 256 + wave * 64 < kUnits && j * 256 + tid < kUnits) {
        const unsigned char *src;
        if (inside) {
          dma16(base, unit_byte[j], stage + 16 * (j * 256 + wave * 64));
        } else {
          const long row = min(max(r_first + static_cast<long>(unit_row[j]), 0L),
                               static_cast<long>(L) - 1);
          src = p_block + static_cast<size_t>(row) * cols3 * sizeof(T) +
                (unit_byte[j] - unit_row[j] * cols3 * sizeof(T));
          dma16(src, stage + 16 * (j * 256 + wave * 64));
        }
      }
    }
  };
  // Six projection values of row i (0 .. kStageRows-1) of a stage.
  auto stage_row = [&](int step, int i, PairRow<T> &dst) {
    const uint32_t *src = reinterpret_cast<const uint32_t *>(
        p_s[step % kStages] + i * kRowBytes + 2 * pair * 3 * sizeof(T));
#pragma unroll
    for (int w = 0; w < PairRow<T>::kWords; ++w)
      dst.word[w] = src[w];
  };
  // Rows before 0 (first segment, first step) come from the short history.
  auto history_row = [&](long row, PairRow<T> &dst) {
    const long hrow = static_cast<long>(short_len - 1) + row;
#pragma unroll
    for (int i = 0; i < PairRow<T>::kWords; ++i)
      dst.word[i] = 0;
    if (short_history != nullptr && hrow >= 0) {
      float v[6];
#pragma unroll
      for (int col = 0; col < 6; ++col)
        v[col] = short_history[static_cast<size_t>(hrow) * cols3 + 3 * cp + col];
      if constexpr (sizeof(T) == 2) {
        // BF16 inputs: the history holds BF16 values.
#pragma unroll
        for (int i = 0; i < 3; ++i)
          dst.word[i] = (__builtin_bit_cast(uint32_t, v[2 * i]) >> 16) |
                        (__builtin_bit_cast(uint32_t, v[2 * i + 1]) & 0xffff0000U);
      } else {
#pragma unroll
        for (int i = 0; i < 6; ++i)
          dst.word[i] = __builtin_bit_cast(uint32_t, v[i]);
      }
    }
  };

  // ---- MFMA lane: channel slice `wave`, fragment group g.
  const int col = lane & 15, g = lane >> 4;
  const size_t cw = c0 + 16 * wave + col;
  const float *h = filter + ((c0 + 16 * wave) / group_size) * k;
  // The wave's filter (k <= 128 taps of its group) goes to LDS between 160
  // zeros on either side, so that the Toeplitz fragments gather from there
  // after the first barrier with unconditional reads (80 taps per lane read
  // from global memory one by one took ~12 us of L2 latency, and conditional
  // LDS reads ~5 us). With 16-byte aligned taps and direct terms both arrive
  // by DMA ahead of the projection stages, so that the first barrier's wait
  // covers them; otherwise by plain loads before the stages are issued (a
  // wait for a load issued behind the DMA would wait for the DMA too). The
  // scratch is the third x2 / y buffer, which the production first writes in
  // phase 1: 448 floats per wave, then the block's 64 direct terms.
  constexpr int kTapPad = 160;
  float *taps_s = &xy_s[2][0][0] + wave * (2 * kTapPad + 128);
  float *direct_s = &xy_s[2][0][0] + 4 * (2 * kTapPad + 128);
  const bool dma_consts = k % 4 == 0 && reinterpret_cast<uintptr_t>(filter) % 16 == 0 &&
                          reinterpret_cast<uintptr_t>(direct) % 16 == 0;
  for (int i = lane; i < kTapPad; i += 64)
    taps_s[i] = 0.0F;
  for (int i = kTapPad + k + lane; i < 2 * kTapPad + 128; i += 64)
    taps_s[i] = 0.0F;
  float d = 0.0F;
  if (dma_consts) {
    if (lane < k / 4)
      dma16(h + 4 * lane, taps_s + kTapPad);
    if (wave == 0 && lane < kMsChannels / 4)
      dma16(direct + c0 + 4 * lane, direct_s);
  } else {
    for (int i = lane; i < k; i += 64)
      taps_s[kTapPad + i] = h[i];
    d = direct[cw];
    asm volatile("" : "+v"(d));
  }
  for (int step = 0; step < kStages && step < steps; ++step)
    issue(step);
  u32x4 a[2][kMsK];
  u32x4 ring_hi[kMsK], ring_lo[kMsK];  // BF16 x 8 fragments as raw words
#pragma unroll
  for (int q = 0; q < kMsK; ++q) {
    // Window rows before the first step (only the first segment has them:
    // u rows -128 .. -1 from the inner history; others start at zero). At
    // step 0 window slot q is register q + 1 (slot 4, register 0, receives
    // step 0), so register q holds rows of step q - 1 relative to the first
    // window.
    uint16_t hi[8] = {}, lo[8] = {};
    if (lead == 0 && inner_history != nullptr && q > 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const long row = 32 * q + 8 * g + e - 160;
        const long hrow = static_cast<long>(k - 1) + row;
        const float u = hrow >= 0 ? inner_history[static_cast<size_t>(hrow) * W + cw] : 0.0F;
        hi[e] = f32_to_bf16(u);
        lo[e] = f32_to_bf16(u - bf16_to_f32(hi[e]));
      }
    }
    ring_hi[q] = __builtin_bit_cast(u32x4, hi);
    ring_lo[q] = __builtin_bit_cast(u32x4, lo);
  }

  // ---- Production of step `step`: rows t_start + 32 step + 4 rg .. + 3
  // from its stage (complete: waited for before the last barrier), u into
  // u_s[step % 2] and x2 into xy_s[step % 3].
  constexpr int kUPlane = kMsChannels * kMsUStride;  // BF16 per u plane
  const int x2_lane = 4 * rg * kMsChannels + 2 * pair;
  const int u_prod[2] = {2 * pair * kMsUStride + ms_ucol(2 * pair, 4 * rg),
                         (2 * pair + 1) * kMsUStride + ms_ucol(2 * pair + 1, 4 * rg)};
  auto produce = [&](int step) __attribute__((always_inline)) {
    PairRow<T> cur[kRows];
    const long first_row = static_cast<long>(t_start) + step * kMsStep + 4 * rg - (kWin - 1);
    if (static_cast<long>(t_start) + step * kMsStep >= kWin - 1) {
#pragma unroll
      for (int i = 0; i < kRows; ++i)
        stage_row(step, 4 * rg + i, cur[i]);
    } else {
#pragma unroll
      for (int i = 0; i < kRows; ++i) {
        if (first_row + i >= 0)
          stage_row(step, 4 * rg + i, cur[i]);
        else
          history_row(first_row + i, cur[i]);
      }
    }
    float *x2 = &xy_s[step % 3][0][0] + x2_lane;
    uint16_t *uplanes = &u_s[step & 1][0][0][0];
    float u[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float fir[6];
#pragma unroll
      for (int c6 = 0; c6 < 6; ++c6) {
        float total = 0.0F;
#pragma unroll
        for (int i = 0; i < kWin; ++i)
          total += cur[j + i].at(c6) * stap[c6][i];
        fir[c6] = total;
      }
      u[0][j] = fir[1] * fir[2];
      u[1][j] = fir[4] * fir[5];
      *reinterpret_cast<float2 *>(x2 + j * kMsChannels) = make_float2(fir[0], fir[3]);
    }
    // Rows (0, 1) and (2, 3) of a channel pack into one word per plane.
    uint32_t uh[2][2], ul[2][2];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        uh[ch][w] = pack_bf16(u[ch][2 * w], u[ch][2 * w + 1]);
        ul[ch][w] = pack_bf16(u[ch][2 * w] - __builtin_bit_cast(float, uh[ch][w] << 16),
                              u[ch][2 * w + 1] - __builtin_bit_cast(float, uh[ch][w] & 0xffff0000U));
      }
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      *reinterpret_cast<uint2 *>(uplanes + u_prod[ch]) = make_uint2(uh[ch][0], uh[ch][1]);
      *reinterpret_cast<uint2 *>(uplanes + kUPlane + u_prod[ch]) =
          make_uint2(ul[ch][0], ul[ch][1]);
    }
  };

  // ---- Products of step `step`: ring update from u_s[step % 2]; when the
  // step emits, Y = T . U and y = x2 * (Y + d u) in place of x2.
  const int ch = 16 * wave + col;
  // Per-lane LDS offsets, fixed for the walk: the ring fragment (rows 8g ..
  // 8g+7 of channel ch), the epilogue's u rows 16 half + 4g .. + 3, and y.
  const int u_ring = ch * kMsUStride + ms_ucol(ch, 8 * g);
  const int u_epi[2] = {ch * kMsUStride + ms_ucol(ch, 4 * g),
                        ch * kMsUStride + ms_ucol(ch, 16 + 4 * g)};
  const int y_lane = 4 * g * kMsChannels + ch;
  // The ring is rotated, not shifted: at step s the window slot q (0 oldest
  // .. kMsK-1 newest) is register (q + s + 1) % kMsK, and the new fragment
  // replaces the oldest. `rot` = (s + 1) % kMsK is a compile-time constant of
  // the unrolled step loop.
  auto multiply = [&](auto rot, int step) __attribute__((always_inline)) {
    constexpr int kRot = decltype(rot)::value;
    const uint16_t *uplanes = &u_s[step & 1][0][0][0];
    ring_hi[(kMsK - 1 + kRot) % kMsK] = *reinterpret_cast<const u32x4 *>(uplanes + u_ring);
    ring_lo[(kMsK - 1 + kRot) % kMsK] =
        *reinterpret_cast<const u32x4 *>(uplanes + kUPlane + u_ring);
    if (step < lead)
      return;
    // Two independent accumulator chains, interleaved.
    f32x4 accs[2] = {{0.0F, 0.0F, 0.0F, 0.0F}, {0.0F, 0.0F, 0.0F, 0.0F}};
#pragma unroll
    for (int q = 0; q < kMsK; ++q)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const bf16x8 t = __builtin_bit_cast(bf16x8, a[half][q]);
        accs[half] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            t, __builtin_bit_cast(bf16x8, ring_hi[(q + kRot) % kMsK]), accs[half], 0, 0, 0);
        accs[half] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            t, __builtin_bit_cast(bf16x8, ring_lo[(q + kRot) % kMsK]), accs[half], 0, 0, 0);
      }
    float *xy = &xy_s[step % 3][0][0] + y_lane;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const f32x4 acc = accs[half];
      const uint2 uhi = *reinterpret_cast<const uint2 *>(uplanes + u_epi[half]);
      const uint2 ulo = *reinterpret_cast<const uint2 *>(uplanes + kUPlane + u_epi[half]);
      const uint32_t hw[4] = {uhi.x << 16, uhi.x & 0xffff0000U, uhi.y << 16, uhi.y & 0xffff0000U};
      const uint32_t lw[4] = {ulo.x << 16, ulo.x & 0xffff0000U, ulo.y << 16, ulo.y & 0xffff0000U};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float total =
            acc[e] + d * (__builtin_bit_cast(float, hw[e]) + __builtin_bit_cast(float, lw[e]));
        xy[(16 * half + e) * kMsChannels] *= total;
      }
    }
  };
  // Flush lane: row tid / 8 of the step, channels (tid % 8) * 8 .. + 7; its
  // output index advances by one step of rows per flushed step.
  const int frow = tid >> 3, fpart = tid & 7;
  size_t flush_index = (t0 + frow) * W + c0 + fpart * 8;
  uint32_t flush_r0 = 0;
  auto flush = [&](int step) __attribute__((always_inline)) {
    if (step >= lead) {
      if (flush_r0 + frow < seg_rows)
        MsOut<O>::flush(&xy_s[step % 3][frow][fpart * 8], out, flush_index);
      flush_index += static_cast<size_t>(kMsStep) * W;
      flush_r0 += kMsStep;
    }
  };

  // Prologue: stage 0 (younger: the DMA of stage 1) and the filter in LDS,
  // the fragments, production of step 0, then stage 1 complete.
  if (steps > 1)
    wait_dma<kDmaMin>();
  else
    wait_dma<0>();
  __syncthreads();
  if (dma_consts)
    d = direct_s[16 * wave + col];
  // Keep d in a register: a load re-issued inside the step loop would make
  // the wait for it also wait for every DMA in flight.
  asm volatile("" : "+v"(d));
  // The taps are BF16 values, so T has no lo plane.
#pragma unroll
  for (int half = 0; half < 2; ++half)
#pragma unroll
    for (int q = 0; q < kMsK; ++q) {
      uint16_t taps[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 32 * q + 8 * g + e;
        const int o = i - 16 * half - col - 128 + (k - 1);  // -160 <= o < k + 31
        taps[e] = f32_to_bf16(taps_s[kTapPad + (causal ? k - 1 - o : o)]);
      }
      a[half][q] = __builtin_bit_cast(u32x4, taps);
    }
  produce(0);
  wait_dma<0>();
  __syncthreads();

  // Phase s: flush s - 1; DMA of step s + 2 into the stage step s used;
  // produce s + 1; multiply s. Before the barrier, the DMA of step s + 2 must
  // be complete (nothing younger is in flight). The flush goes out ahead of
  // the DMA: the other order, with the wait leaving the younger flush
  // stores in flight, measured 1 % slower.
  auto phase = [&](auto rot, int step) __attribute__((always_inline)) {
    if (step >= 1)
      flush(step - 1);
    if (step + 2 < steps)
      issue(step + 2);
    if (step + 1 < steps)
      produce(step + 1);
    multiply(rot, step);
    if (step + 2 < steps)
      wait_dma<0>();
    __syncthreads();
  };
  // Unrolled by the ring length so that the rotation is static.
  for (int step = 0; step < steps; step += kMsK) {
    phase(std::integral_constant<int, 1>{}, step);
    if (step + 1 < steps)
      phase(std::integral_constant<int, 2>{}, step + 1);
    if (step + 2 < steps)
      phase(std::integral_constant<int, 3>{}, step + 2);
    if (step + 3 < steps)
      phase(std::integral_constant<int, 4>{}, step + 3);
    if (step + 4 < steps)
      phase(std::integral_constant<int, 0>{}, step + 4);
  }
  flush(steps - 1);
}

// ---- HCL (modal long filter) in one pass on MFMA.
// Per channel c (modes m < 16: pole p_m, residue R_m, direct D) and 16-row
// block b with inputs u_{16b+j}, the recurrence s_t = p s_{t-1} + u_t,
// y_t = sum_m R_m s_t + D u_t becomes three 16 x 16 products:
//   Z = W U          W[m][j] = p_m^(15-j)        local block-end states
//   S_b = p^16 S_{b-1} + Z_b                     a 16-lane scan over blocks
//   Y = H U + V S'   H[r][j] = h[r-j] (j <= r) + D [j = r], h[n] = sum_m R_m p_m^n,
//                    V[r][m] = R_m p_m^(r+1), S'_b = S_{b-1}
// with U[j][b] = u_{16b+j} of one channel as the B operand, so one
// v_mfma_f32_16x16x16_bf16 covers 256 rows of a channel. Each product runs
// on split BF16 planes (hi*hi + hi*lo + lo*hi), the scan in F32.
// A block owns 16 channels and walks the whole sequence in steps of kStep
// rows (256 for BF16 projections, 128 for F32), so the projection is read
// once and the modal state never leaves the block: production (short FIR,
// gates, u as split planes into LDS [channel][row], x2 into LDS [row][ch])
// from DMA-staged projection rows, the products (wave w: channels 2w, 2w+1;
// y = x2 * Y in place of x2), and a flush of whole 16-channel rows, software
// pipelined as in the HCM stream kernel (phase s: flush s-1, produce s+1,
// multiply s). Consecutive channel groups are placed on one XCD, so the
// four blocks that share each 128-byte line of a projection or output row
// meet in one L2.
// 16 channels per block (8 per block, two blocks per CU: 82 -> 83 us with
// BF16 output, 98 -> 149 us with split planes, whose 16-byte row pieces
// the L2 merges badly).
constexpr int kHmChannels = 16;
constexpr int kHmPairs = kHmChannels / 2;      // production channel pairs
constexpr int kHmFlushParts = kHmChannels / 8; // flush lanes per row
// Wave roles. With kRoles, 4 producer waves (DMA and production, two row
// groups per lane) and 8 consumer waves (two channels each: products, scan,
// gate, flush), three waves per SIMD: 80 -> 70 us at config 2 with BF16
// output. Split-plane output keeps 8 waves that each do both (with roles its
// projection reads were fetched 1.4x from HBM, the L2 losing the lines that
// neighbouring blocks share before they read them: 98 -> 120 us).
template <bool kRoles> struct HmRoles {
  static constexpr int kProducerWaves = kRoles ? 4 : kHmChannels / 2;
  static constexpr int kThreads = 64 * (kRoles ? 4 + kHmChannels / 2 : kHmChannels / 2);
  static constexpr int kProducers = 64 * kProducerWaves;
  static constexpr int kTasks = 64 * kHmPairs / kProducers;  // row groups per producer lane
};
template <typename O> constexpr bool kHmRoles = !std::is_same<O, SplitOut>::value;
template <typename O> constexpr int kHmThreads = HmRoles<kHmRoles<O>>::kThreads;

template <typename T, int kProducers> struct HmShape {
  static constexpr int kStep = sizeof(T) == 2 ? 256 : 128;   // rows per step
  static constexpr int kBlocks = kStep / 16;                 // MFMA columns used
  static constexpr int kWin = 3;                             // short FIR length
  static constexpr int kRowBytes = kHmChannels * 3 * static_cast<int>(sizeof(T));
  static constexpr int kStageRows = kStep + kWin - 1;
  static constexpr int kStageBytes = kStageRows * kRowBytes;
  static constexpr int kUnitsPerRow = kRowBytes / 16;
  static constexpr int kUnits = kStageBytes / 16;
  static constexpr int kDma = (kUnits + kProducers - 1) / kProducers;
  static constexpr int kRowsPerThread = kStep / 64;           // production
  // u stage [channel][row] (BF16) and x2 / y stage [channel][row] (F32):
  // row r sits at hm_upos(r) / hm_ypos(r), which pad 8 BF16 every 128 rows
  // and 4 floats every 64 rows, so that the product lanes' 16 blocks (rows
  // 16 b + 4 g) fall on distinct bank groups; the strides keep the
  // production lanes' writes (8 channel pairs x 4-row groups) distinct too.
  static constexpr int kUStride = sizeof(T) == 2 ? 280 : 136;
  static constexpr int kFlushTasks = kStep * kHmFlushParts;   // 8 channels each
  // x2 / y stage [channel][row]: a product lane's four rows are one 16-byte
  // access, and the stride puts the two 8-channel halves of the flush 32
  // banks apart.
  static constexpr int kYStride = kStep + 4 * (kStep / 64) + 4;
};

typedef short hm_s4 __attribute__((ext_vector_type(4)));
constexpr int kHmStages = 3;
__device__ inline int hm_upos(int row) { return row + 8 * (row >> 7); }
__device__ inline int hm_ypos(int row) { return row + 4 * (row >> 6); }
// Phase variants of the HCL kernel: the first step (rows before 0 from the
// short history), any step (every bound checked), and the interior steps,
// whose rows, DMA and flush all lie inside the sequence (no checks, so the
// whole phase is one basic block the compiler can schedule across).
constexpr int kHmGeneric = 0, kHmFirst = 1, kHmSteady = 2;
template <int kMode> using HmMode = std::integral_constant<int, kMode>;

// s_waitcnt vmcnt(n) for a run-time n (wave-uniform, 0 .. 9).
__device__ inline void hm_wait(int n) {
  switch (n) {
    case 0: wait_dma<0>(); break;
    case 1: wait_dma<1>(); break;
    case 2: wait_dma<2>(); break;
    case 3: wait_dma<3>(); break;
    case 4: wait_dma<4>(); break;
    case 5: wait_dma<5>(); break;
    case 6: wait_dma<6>(); break;
    case 7: wait_dma<7>(); break;
    case 8: wait_dma<8>(); break;
    default: wait_dma<9>(); break;
  }
}

// Split of four values into BF16 hi / lo fragments.
__device__ inline void hm_split4(const float (&v)[4], hm_s4 &hi, hm_s4 &lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t h = f32_to_bf16(v[i]);
    hi[i] = static_cast<short>(h);
    lo[i] = static_cast<short>(f32_to_bf16(v[i] - bf16_to_f32(h)));
  }
}
// x^n (0 <= n < 32) by repeated squaring.
__device__ inline double hm_pow(double x, int n) {
  double r = 1.0;
#pragma unroll
  for (int bit = 0; bit < 5; ++bit) {
    if (n & (1 << bit))
      r *= x;
    x *= x;
  }
  return r;
}
// Value of lane l - d within its row of 16 lanes (0 for the first d lanes).
template <int kD> __device__ inline float hm_shift(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, v), 0x110 + kD, 0xf, 0xf, true));
}
// One level of the block scan over eight chains: v += q * v[lane - kD]
// (nothing for the first kD lanes of each row of 16), as v_fmac_f32 with a
// DPP row shift on the multiplicand: one instruction per chain instead of a
// DPP move and an FMA. Same single rounding as fmaf(q, shifted v, v). The
// s_nop gives the two wait states a DPP read needs after the VALU write of
// its source, which the compiler cannot see inside the asm; the sources must
// be VALU results (not MFMA results, which need more).
template <int kD> __device__ inline void hm_scan_level(float (&v)[2][4], const float (&qa)[4],
                                                       const float (&qb)[4]) {
  asm(
      "s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %0, %8 row_shr:%c16 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %1, %1, %9 row_shr:%c16 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %2, %2, %10 row_shr:%c16 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %3, %3, %11 row_shr:%c16 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %4, %4, %12 row_shr:%c16 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %5, %5, %13 row_shr:%c16 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %6, %6, %14 row_shr:%c16 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %7, %7, %15 row_shr:%c16 row_mask:0xf bank_mask:0xf bound_ctrl:1"
      : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[0][2]), "+v"(v[0][3]), "+v"(v[1][0]),
        "+v"(v[1][1]), "+v"(v[1][2]), "+v"(v[1][3])
      : "v"(qa[0]), "v"(qa[1]), "v"(qa[2]), "v"(qa[3]), "v"(qb[0]), "v"(qb[1]), "v"(qb[2]),
        "v"(qb[3]), "n"(kD));
}
__device__ inline f32x4 hm_mfma3(const hm_s4 &ah, const hm_s4 &al, const hm_s4 &bh,
                                 const hm_s4 &bl, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bl, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al, bh, acc, 0, 0, 0);
  return acc;
}

// Output of 8 channels of one row (16- or 32-byte pieces). Plain stores,
// unlike the stream kernels' non-temporal ones: a block writes only 32 bytes
// of each 128-byte output line, and the L2 merges the four blocks' pieces
// into whole lines before they reach HBM.
template <typename O> struct HmOut;
template <> struct HmOut<float *> {
  __device__ static int stores(float *) { return 2; }
  __device__ static void put(const float (&v)[8], float *out, size_t index) {
    *reinterpret_cast<f32x4 *>(out + index) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4 *>(out + index + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
};
template <typename O> struct HmOut16 {
  __device__ static int stores(const O &) { return 1; }
  __device__ static void put(const float (&v)[8], const O &out, size_t index) {
    note_eight(Plane16<O>::flag(out), v);
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = Plane16<O>::pack(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4 *>(Plane16<O>::ptr(out) + index) = w;
  }
};
template <> struct HmOut<uint16_t *> : HmOut16<uint16_t *> {};
template <> struct HmOut<F16Out> : HmOut16<F16Out> {};
template <> struct HmOut<SplitOut> {
  __device__ static int stores(const SplitOut &out) { return out.lo != nullptr ? 2 : 1; }
  __device__ static void put(const float (&v)[8], const SplitOut &out, size_t index) {
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hi[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
      lo[i] = pack_bf16(v[2 * i] - __builtin_bit_cast(float, hi[i] << 16),
                        v[2 * i + 1] - __builtin_bit_cast(float, hi[i] & 0xffff0000U));
    }
    *reinterpret_cast<u32x4 *>(out.hi + index) = u32x4{hi[0], hi[1], hi[2], hi[3]};
    if (out.lo != nullptr)
      *reinterpret_cast<u32x4 *>(out.lo + index) = u32x4{lo[0], lo[1], lo[2], lo[3]};
  }
};

template <typename T, typename O>
__global__ __launch_bounds__(kHmThreads<O>, 1) void hcl_mfma_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, size_t L, size_t W,
    const float *__restrict__ poles, const float *__restrict__ residues,
    const float *__restrict__ direct, int S, float *__restrict__ modal_state, O out) {
  constexpr bool kRoles = kHmRoles<O>;
  using Roles = HmRoles<kRoles>;
  constexpr int kHmProducers = Roles::kProducers, kHmTasks = Roles::kTasks;
  using Shape = HmShape<T, kHmProducers>;
  constexpr int kStep = Shape::kStep, kWin = Shape::kWin, kPR = Shape::kRowsPerThread;
  __shared__ __attribute__((aligned(16))) unsigned char p_s[kHmStages][Shape::kStageBytes];
  __shared__ __attribute__((aligned(16))) uint16_t u_s[2][2][kHmChannels][Shape::kUStride];
  __shared__ __attribute__((aligned(16))) float xy_s[3][kHmChannels][Shape::kYStride];

  const unsigned groups = static_cast<unsigned>(W / kHmChannels);
  const unsigned xcd = blockIdx.x % 8, per_xcd = groups / 8, extra = groups % 8;
  const size_t c0 =
      static_cast<size_t>(xcd * per_xcd + min(xcd, extra) + blockIdx.x / 8) * kHmChannels;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool producer = !kRoles || wave < Roles::kProducerWaves;
  const bool consumer = !kRoles || !producer;
  const size_t cols3 = 3 * W;
  const int steps = static_cast<int>((L + kStep - 1) / kStep);

  // ---- DMA of the projection rows of step `step` (rows 32 step - 2 ..):
  // rows clamp to [0, L); rows before 0 come from the short history, rows
  // past L feed only outputs that are dropped (their u is zeroed).
  const unsigned char *p_block = reinterpret_cast<const unsigned char *>(P + 3 * c0);
  uint32_t unit_byte[Shape::kDma];
#pragma unroll
  for (int j = 0; j < Shape::kDma; ++j) {
    const int unit = min(j * kHmProducers + tid, Shape::kUnits - 1);
    unit_byte[j] = static_cast<uint32_t>(unit / Shape::kUnitsPerRow * cols3 * sizeof(T) +
                                         16 * (unit % Shape::kUnitsPerRow));
  }
  auto issue = [&](int step, auto steady) __attribute__((always_inline)) {
    const long r_first = static_cast<long>(step) * kStep - (kWin - 1);
    unsigned char *stage = p_s[step % kHmStages];
    // Steps whose rows all lie in [0, L) use a uniform base and fixed
    // per-lane offsets; the first and last steps clamp each row.
    const bool inside = decltype(steady)::value ||
                        (r_first >= 0 && r_first + Shape::kStageRows <= static_cast<long>(L));
    const unsigned char *base =
        p_block + static_cast<size_t>(max(r_first, 0L)) * cols3 * sizeof(T);
#pragma unroll
    for (int j = 0; j < Shape::kDma; ++j) {
      if (j * kHmProducers + wave * 64 < Shape::kUnits &&
          j * kHmProducers + tid < Shape::kUnits) {
        if (inside) {
          dma16(base, unit_byte[j], stage + 16 * (j * kHmProducers + wave * 64));
        } else {
          const int unit = j * kHmProducers + tid;
          const long row = min(max(r_first + unit / Shape::kUnitsPerRow, 0L),
                               static_cast<long>(L) - 1);
          dma16(p_block + static_cast<size_t>(row) * cols3 * sizeof(T) +
                    16 * (unit % Shape::kUnitsPerRow),
                stage + 16 * (j * kHmProducers + wave * 64));
        }
      }
    }
  };

  // ---- Production lane (producer waves): channels 2 pr, 2 pr + 1 and, for
  // each task t, rows kPR rg .. + kPR-1 of row group rg = rg0 + t 64 / kHmTasks.
  const int pr = tid % kHmPairs, rg0 = (tid % kHmProducers) / kHmPairs;
  const size_t cp = c0 + 2 * pr;
  float stap[6][kWin];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch) {
    float t3[3][kWin];
    load_window_taps(short_filter, kWin, cp + ch, t3);
#pragma unroll
    for (int s = 0; s < 3; ++s)
#pragma unroll
      for (int i = 0; i < kWin; ++i)
        stap[3 * ch + s][i] = t3[s][i];
  }
  auto stage_row = [&](int step, int i, PairRow<T> &dst) {
    const uint32_t *src = reinterpret_cast<const uint32_t *>(
        p_s[step % kHmStages] + i * Shape::kRowBytes + 2 * pr * 3 * sizeof(T));
#pragma unroll
    for (int w = 0; w < PairRow<T>::kWords; ++w)
      dst.word[w] = src[w];
  };
  auto history_row = [&](long row, PairRow<T> &dst) {  // row in [-2, -1]
    const long hrow = static_cast<long>(kWin - 1) + row;
#pragma unroll
    for (int i = 0; i < PairRow<T>::kWords; ++i)
      dst.word[i] = 0;
    if (short_history != nullptr) {
      float v[6];
#pragma unroll
      for (int col = 0; col < 6; ++col)
        v[col] = short_history[static_cast<size_t>(hrow) * cols3 + 3 * cp + col];
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
          dst.word[i] = (__builtin_bit_cast(uint32_t, v[2 * i]) >> 16) |
                        (__builtin_bit_cast(uint32_t, v[2 * i + 1]) & 0xffff0000U);
      } else {
#pragma unroll
        for (int i = 0; i < 6; ++i)
          dst.word[i] = __builtin_bit_cast(uint32_t, v[i]);
      }
    }
  };
  // Only step 0 reads rows before 0 (from the short history): the steady
  // state has no global loads here, so the compiler's wait for their data
  // cannot stall the DMA and store streams of the main loop.
  // Production in two parts (the phase issues every LDS read first): the
  // staged rows of the lane's window, then the arithmetic and the LDS writes.
  PairRow<T> cur_rows[kHmTasks][kPR + kWin - 1];
  auto produce_load_task = [&](int step, auto mode, int t) __attribute__((always_inline)) {
    const int rg = rg0 + t * (64 / kHmTasks);
    const long first = static_cast<long>(step) * kStep + kPR * rg - (kWin - 1);
#pragma unroll
    for (int i = 0; i < kPR + kWin - 1; ++i) {
      if (decltype(mode)::value != kHmFirst || first + i >= 0)
        stage_row(step, kPR * rg + i, cur_rows[t][i]);
      else
        history_row(first + i, cur_rows[t][i]);
    }
  };
  auto produce_task = [&](int step, auto mode, int t) __attribute__((always_inline)) {
    const int rg = rg0 + t * (64 / kHmTasks);
    const PairRow<T> (&cur)[kPR + kWin - 1] = cur_rows[t];
    const long first = static_cast<long>(step) * kStep + kPR * rg - (kWin - 1);
    float u[2][kPR], x2[2][kPR];
#pragma unroll
    for (int j = 0; j < kPR; ++j) {
      float fir[6];
#pragma unroll
      for (int c6 = 0; c6 < 6; ++c6) {
        float total = 0.0F;
#pragma unroll
        for (int i = 0; i < kWin; ++i)
          total += cur[j + i].at(c6) * stap[c6][i];
        fir[c6] = total;
      }
      const bool valid = decltype(mode)::value == kHmSteady ||
                         first + kWin - 1 + j < static_cast<long>(L);
      u[0][j] = valid ? fir[1] * fir[2] : 0.0F;
      u[1][j] = valid ? fir[4] * fir[5] : 0.0F;
      x2[0][j] = fir[0];
      x2[1][j] = fir[3];
    }
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      float *dst = &xy_s[step % 3][2 * pr + ch][hm_ypos(kPR * rg)];
      if constexpr (kPR == 4)
        *reinterpret_cast<f32x4 *>(dst) = f32x4{x2[ch][0], x2[ch][1], x2[ch][2], x2[ch][3]};
      else
        *reinterpret_cast<float2 *>(dst) = make_float2(x2[ch][0], x2[ch][1]);
    }
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      uint32_t hi[kPR / 2], lo[kPR / 2];
#pragma unroll
      for (int w = 0; w < kPR / 2; ++w) {
        hi[w] = pack_bf16(u[ch][2 * w], u[ch][2 * w + 1]);
        lo[w] = pack_bf16(u[ch][2 * w] - __builtin_bit_cast(float, hi[w] << 16),
                          u[ch][2 * w + 1] - __builtin_bit_cast(float, hi[w] & 0xffff0000U));
      }
      uint16_t *dst_hi = &u_s[step & 1][0][2 * pr + ch][hm_upos(kPR * rg)];
      uint16_t *dst_lo = &u_s[step & 1][1][2 * pr + ch][hm_upos(kPR * rg)];
      if constexpr (kPR == 4) {
        *reinterpret_cast<uint2 *>(dst_hi) = make_uint2(hi[0], hi[1]);
        *reinterpret_cast<uint2 *>(dst_lo) = make_uint2(lo[0], lo[1]);
      } else {
        *reinterpret_cast<uint32_t *>(dst_hi) = hi[0];
        *reinterpret_cast<uint32_t *>(dst_lo) = lo[0];
      }
    }
  };
  auto produce = [&](int step, auto mode) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < kHmTasks; ++t) {
      produce_load_task(step, mode, t);
      produce_task(step, mode, t);
    }
  };

  // ---- Product lane: channels 2 wave + k (k = 0, 1); column (block) b,
  // fragment group g. The constant fragments are computed once per channel
  // in double precision, and the filter h[n] = sum_m R_m p_m^n by four lanes
  // per n (modes 4g .. 4g+3 each) reduced across the lane groups. The loads
  // are issued here; the arithmetic (`constants`) runs after the first
  // barrier, beside the production of step 0.
  const int b = lane & 15, g = lane >> 4;
  const int cwave = !kRoles ? wave : producer ? 0 : wave - Roles::kProducerWaves;
  hm_s4 w_hi[2], w_lo[2], h_hi[2], h_lo[2], v_hi[2], v_lo[2];
  float q1[2][4], q2[2][4], q4[2][4], q8[2][4], qb[2][4], carry[2][4];
  // p of mode b, p and R of modes 4g + v, and D of each channel.
  float p_b[2], p_g[2][4], r_g[2][4], d_c[2];
#pragma unroll
  for (int k = 0; k < 2 && consumer; ++k) {
    const size_t c = c0 + 2 * cwave + k;
    p_b[k] = b < S ? poles[c * S + b] : 0.0F;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * g + v;
      p_g[k][v] = m < S ? poles[c * S + m] : 0.0F;
      r_g[k][v] = m < S ? residues[c * S + m] : 0.0F;
      carry[k][v] = (modal_state != nullptr && m < S) ? modal_state[c * S + m] : 0.0F;
    }
    d_c[k] = direct[c];
  }
  // Powers with shared factors: p_g^b serves h[b], V (R p^(b+1)) and the
  // lane's block multiplier q^(b+1) = (p^b)^16 p^16; W's four powers of p_b
  // are one power and three products.
  auto constants = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      double pgb[4], term[4];
      double h_part = 0.0;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        pgb[v] = hm_pow(p_g[k][v], b);
        term[v] = static_cast<double>(r_g[k][v]) * pgb[v];
        h_part += term[v];
      }
      float h_n = static_cast<float>(h_part);
      h_n += __shfl_xor(h_n, 16);
      h_n += __shfl_xor(h_n, 32);
      const double pb = p_b[k];
      double wd[4];
      wd[3] = hm_pow(pb, 12 - 4 * g);  // K index j = 4g + v takes pb^(15 - j)
      wd[2] = wd[3] * pb;
      wd[1] = wd[2] * pb;
      wd[0] = wd[1] * pb;
      float wv[4], hv[4], vv[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int j = 4 * g + v;  // A-operand K index; the A row is b
        wv[v] = static_cast<float>(wd[v]);
        const float h = __shfl(h_n, (b - j) & 15);
        hv[v] = j <= b ? (j == b ? static_cast<float>(static_cast<double>(h) + d_c[k]) : h)
                       : 0.0F;
        const double p = p_g[k][v];
        vv[v] = static_cast<float>(term[v] * p);
        double q = p * p;  // block multiplier p^16 of mode 4g + v
        q *= q;
        q *= q;
        q *= q;
        const double q2d = q * q, q4d = q2d * q2d;
        q1[k][v] = static_cast<float>(q);
        q2[k][v] = static_cast<float>(q2d);
        q4[k][v] = static_cast<float>(q4d);
        q8[k][v] = static_cast<float>(q4d * q4d);
        double x = pgb[v] * pgb[v];
        x *= x;
        x *= x;
        x *= x;
        qb[k][v] = static_cast<float>(x * q);
      }
      hm_split4(wv, w_hi[k], w_lo[k]);
      hm_split4(hv, h_hi[k], h_lo[k]);
      hm_split4(vv, v_hi[k], v_lo[k]);
    }
  };

  float sp_last[2][4];
  // The products of step `step` in two parts, so the phase can run the
  // production of the next step between them: part one reads U and issues
  // Z = W U and H U for both channels (the matrix cores work while the
  // production's VALU runs); part two scans Z (eight independent chains per
  // lane: two channels x four modes), adds V S' and applies the gate.
  hm_s4 ub_hi[2], ub_lo[2];
  f32x4 z_acc[2], y_acc[2], x2_frag[2];
  // LDS reads of the products: U of step `step` and its gate x2.
  auto multiply_load = [&](int step) __attribute__((always_inline)) {
    const uint16_t *uh = &u_s[step & 1][0][0][0];
    const uint16_t *ul = &u_s[step & 1][1][0][0];
    const bool col_ok = b < Shape::kBlocks;
    const int row0 = 16 * (col_ok ? b : 0) + 4 * g;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int ch = 2 * cwave + k;
      ub_hi[k] = *reinterpret_cast<const hm_s4 *>(uh + ch * Shape::kUStride + hm_upos(row0));
      ub_lo[k] = *reinterpret_cast<const hm_s4 *>(ul + ch * Shape::kUStride + hm_upos(row0));
      x2_frag[k] = *reinterpret_cast<const f32x4 *>(&xy_s[step % 3][ch][hm_ypos(row0)]);
      if (!col_ok) {
        ub_hi[k] = hm_s4{0, 0, 0, 0};
        ub_lo[k] = hm_s4{0, 0, 0, 0};
      }
    }
  };
  auto multiply_a = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
      z_acc[k] = hm_mfma3(w_hi[k], w_lo[k], ub_hi[k], ub_lo[k], f32x4{0.0F, 0.0F, 0.0F, 0.0F});
#pragma unroll
    for (int k = 0; k < 2; ++k)
      y_acc[k] = hm_mfma3(h_hi[k], h_lo[k], ub_hi[k], ub_lo[k], f32x4{0.0F, 0.0F, 0.0F, 0.0F});
  };
  auto multiply_b = [&](int step) __attribute__((always_inline)) {
    const bool col_ok = b < Shape::kBlocks;
    const int row0 = 16 * (col_ok ? b : 0) + 4 * g;
    // Inclusive scan over the blocks (lanes b of each row of 16), level by
    // level across the eight chains.
    float v[2][4];
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[k][e] = z_acc[k][e];
    // The first level stays compiler-visible: it reads the MFMA results, whose
    // wait states the compiler inserts.
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[k][e] = fmaf(q1[k][e], hm_shift<1>(v[k][e]), v[k][e]);
    if constexpr (kRoles) {
      hm_scan_level<2>(v, q2[0], q2[1]);
      hm_scan_level<4>(v, q4[0], q4[1]);
      hm_scan_level<8>(v, q8[0], q8[1]);
    } else {
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[k][e] = fmaf(q2[k][e], hm_shift<2>(v[k][e]), v[k][e]);
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[k][e] = fmaf(q4[k][e], hm_shift<4>(v[k][e]), v[k][e]);
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[k][e] = fmaf(q8[k][e], hm_shift<8>(v[k][e]), v[k][e]);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[k][e] = fmaf(qb[k][e], carry[k][e], v[k][e]);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      float sp[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sp[e] = hm_shift<1>(v[k][e]) + (b == 0 ? carry[k][e] : 0.0F);
      hm_s4 s_hi, s_lo;
      hm_split4(sp, s_hi, s_lo);
      y_acc[k] = hm_mfma3(v_hi[k], v_lo[k], s_hi, s_lo, y_acc[k]);
      // Kept for the final modal state (no memory access here: a global load
      // or store in the step loop would make every step wait for the DMA
      // and store streams).
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sp_last[k][e] = sp[e];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        carry[k][e] = __shfl(v[k][e], 16 * g + Shape::kBlocks - 1);
    }
    if (col_ok) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        f32x4 *xy = reinterpret_cast<f32x4 *>(&xy_s[step % 3][2 * cwave + k][hm_ypos(row0)]);
        const f32x4 x2 = x2_frag[k];
        const f32x4 y = y_acc[k];
        *xy = f32x4{x2[0] * y[0], x2[1] * y[1], x2[2] * y[2], x2[3] * y[3]};
      }
    }
  };

  // ---- Flush lane: row fr of a step, channels 8 fh .. 8 fh + 7.
  const int ctid = !kRoles ? tid : producer ? 0 : tid - kHmProducers;
  const bool flusher = consumer && ctid < Shape::kFlushTasks;
  const int fr = ctid / kHmFlushParts, fh = ctid % kHmFlushParts;
  // The flush lane's output index advances by one step of rows per call.
  size_t flush_index = static_cast<size_t>(fr) * W + c0 + 8 * fh;
  size_t flush_row = static_cast<size_t>(fr);
  float flush_v[8];
  auto flush_load = [&](int step) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      flush_v[i] = xy_s[step % 3][8 * fh + i][hm_ypos(fr)];
  };
  auto flush_store = [&](auto steady) __attribute__((always_inline)) {
    if (flusher && (decltype(steady)::value || flush_row < L))
      HmOut<O>::put(flush_v, out, flush_index);
    flush_index += static_cast<size_t>(kStep) * W;
    flush_row += kStep;
  };
  auto flush = [&](int step, auto steady) __attribute__((always_inline)) {
    flush_load(step);
    flush_store(steady);
  };

  // Three projection stages: phase s issues the DMA of step s + 3 and must
  // see step s + 2 landed before its closing barrier. Every producer wave
  // issues at least kDmaMin DMAs per step, so waiting down to that many
  // younger ones is conservative.
  constexpr int kDmaMin = Shape::kUnits / kHmProducers;
  // Phase s: the producers issue the DMA of step s + 3 and produce step
  // s + 1, then wait for the DMA of step s + 2 (younger: the one just
  // issued); the consumers read U and x2 of step s and the y of step s - 1,
  // form the products, write y = x2 Y in place of x2 and store step s - 1.
  // The consumers never wait for their stores, which may stay in flight
  // across barriers. Each role runs its own loop (so that neither holds the
  // other's registers), with the same barriers.
  auto producer_phase = [&](int step, auto steady) __attribute__((always_inline)) {
    constexpr bool kSteady = decltype(steady)::value;
    const bool more = kSteady || step + kHmStages < steps;
    if (more)
      issue(step + kHmStages, steady);
    if (kSteady || step + 1 < steps)
      produce(step + 1, HmMode<kSteady ? kHmSteady : kHmGeneric>{});
    if (kSteady || step + 2 < steps)
      hm_wait(more ? kDmaMin : 0);
    __syncthreads();
  };
  auto consumer_phase = [&](int step, auto steady) __attribute__((always_inline)) {
    const bool flushes = decltype(steady)::value || step >= 1;
    multiply_load(step);
    if (flushes)
      flush_load(step - 1);
    multiply_a();
    multiply_b(step);
    if (flushes)
      flush_store(steady);
    __syncthreads();
  };
  // Interior steps 2 <= step < L / kStep - 3: the DMA of step + 3, the
  // production of step + 1 and the flush of step - 1 lie inside [0, L).
  const int steady_end = static_cast<int>(L / kStep) - 3;
  auto walk = [&](auto role_phase) __attribute__((always_inline)) {
    int step = 0;
    for (; step < steps && step < 2; ++step)
      role_phase(step, std::false_type{});
    for (; step < steady_end; ++step)
      role_phase(step, std::true_type{});
    for (; step < steps; ++step)
      role_phase(step, std::false_type{});
  };
  // Without roles every wave does both, the consumer's LDS reads first, and
  // waits for the DMA of step s + 2 behind this phase's DMA and the flush
  // stores of this and the previous phase (vector memory operations complete
  // in issue order).
  const int stores = flusher ? HmOut<O>::stores(out) : 0;
  auto merged_phase = [&](int step, auto steady) __attribute__((always_inline)) {
    constexpr bool kSteady = decltype(steady)::value;
    const bool more = kSteady || step + kHmStages < steps;
    const bool flushes = kSteady || step >= 1;
    if (more)
      issue(step + kHmStages, steady);
    multiply_load(step);
    if (flushes)
      flush_load(step - 1);
    multiply_a();
    if (kSteady || step + 1 < steps)
      produce(step + 1, HmMode<kSteady ? kHmSteady : kHmGeneric>{});
    multiply_b(step);
    if (flushes)
      flush_store(steady);
    if (kSteady || step + 2 < steps)
      hm_wait((more ? kDmaMin : 0) + (step >= 1 ? stores : 0) + (step >= 2 ? stores : 0));
    __syncthreads();
  };
  if (!kRoles)
    constants();
  if (producer) {
    for (int step = 0; step < kHmStages && step < steps; ++step)
      issue(step, std::false_type{});
    hm_wait(min(steps - 1, kHmStages - 1) * kDmaMin);
  }
  __syncthreads();
  if (producer) {
    produce(0, HmMode<kHmFirst>{});
    hm_wait(steps > 2 ? kDmaMin : 0);
  }
  if (kRoles && consumer)
    constants();  // beside the production of step 0
  __syncthreads();
  if constexpr (kRoles) {
    if (producer) {
      walk(producer_phase);
      return;
    }
    walk(consumer_phase);
  } else {
    walk(merged_phase);
  }
  flush(steps - 1, std::false_type{});
  // State after row L-1: the last step's block bl holds that row at rl;
  // the lanes of column bl continue from S_{bl-1} over rows 0..rl.
  if (modal_state != nullptr) {
    const int step = steps - 1;
    const int rows = static_cast<int>(L - static_cast<size_t>(step) * kStep);
    const int bl = (rows - 1) / 16, rl = (rows - 1) % 16;
    if (b == bl) {
      const uint16_t *uh = &u_s[step & 1][0][0][0];
      const uint16_t *ul = &u_s[step & 1][1][0][0];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int ch = 2 * cwave + k;
        const size_t c = c0 + ch;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 4 * g + e;
          if (m < S) {
            const float pm = poles[c * S + m];
            float st = sp_last[k][e];
            for (int j = 0; j <= rl; ++j) {
              const int at = ch * Shape::kUStride + hm_upos(16 * bl + j);
              st = fmaf(pm, st, bf16_to_f32(uh[at]) + bf16_to_f32(ul[at]));
            }
            modal_state[c * S + m] = st;
          }
        }
      }
    }
  }
}

// Rewrites the inner (u) history with the last k-1 rows of [history ; u].
// Runs after the main kernel and before the short history moves on.
template <typename T>
__global__ void inner_history_kernel(const T *__restrict__ P,
                                     const float *__restrict__ short_history,
                                     const uint16_t *__restrict__ short_filter,
                                     int short_len, size_t L, size_t W, size_t planar,
                                     float *inner_history, int hist) {
  const size_t c = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (c >= W)
    return;
  float taps[3][kMaxShort];
  load_short_taps(short_filter, short_len, c, taps);
  const size_t cols3 = 3 * W;
  // With L >= hist every new row comes from u and rows are independent: one
  // block row per history row. Otherwise rows shift in place, oldest first.
  const int h_begin = gridDim.y > 1 ? static_cast<int>(blockIdx.y) : 0;
  const int h_end = gridDim.y > 1 ? h_begin + 1 : hist;
  for (int h = h_begin; h < h_end; ++h) {
    const long source = static_cast<long>(h) + static_cast<long>(L);  // in [hist ; u]
    float value;
    if (source < hist) {
      value = inner_history[static_cast<size_t>(source) * W + c];
    } else {
      const long t = source - hist;
      float x2, u;
      gates(P, short_history, taps, short_len, cols3, planar, t, c, &x2, &u);
      value = u;
    }
    inner_history[static_cast<size_t>(h) * W + c] = value;
  }
}

// Short continuation (L < hist): history <- last hist rows of [history ; u]
// for 64 channels per block. All old rows that survive are read into LDS
// before any row is rewritten, so every (row, channel) runs in parallel.
template <typename T>
__global__ __launch_bounds__(256) void inner_history_shift_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len, size_t L, size_t W,
    size_t planar, float *inner_history, int hist) {
  extern __shared__ float shift_s[];  // [hist][64]
  const int lane = threadIdx.x & 63;
  const size_t c = blockIdx.x * 64ULL + lane;
  const bool valid = c < W;
  const int keep = hist - static_cast<int>(L);  // rows that move down by L
  for (int h = threadIdx.x >> 6; h < keep; h += 4)
    shift_s[h * 64 + lane] = valid ? inner_history[(h + L) * W + c] : 0.0F;
  __syncthreads();
  if (!valid)
    return;
  float taps[3][kMaxShort];
  load_short_taps(short_filter, short_len, c, taps);
  const size_t cols3 = 3 * W;
  for (int h = threadIdx.x >> 6; h < hist; h += 4) {
    float value;
    if (h < keep) {
      value = shift_s[h * 64 + lane];
    } else {
      float x2;
      gates(P, short_history, taps, short_len, cols3, planar, h - keep, c, &x2, &value);
    }
    inner_history[static_cast<size_t>(h) * W + c] = value;
  }
}

template <typename T>
__global__ void short_history_kernel(const T *__restrict__ P, size_t L,
                                     size_t cols3, float *history, int hist) {
  const size_t c = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (c >= cols3)
    return;
  for (int h = 0; h < hist; ++h) {
    const long source = static_cast<long>(h) + static_cast<long>(L);
    history[static_cast<size_t>(h) * cols3 + c] =
        source < hist ? history[static_cast<size_t>(source) * cols3 + c]
                      : load_act(P, static_cast<size_t>(source - hist) * cols3 + c);
  }
}


// ---- One-row continuation (the decode step) of the whole operator in one
// launch. A block of 1024 threads (16 groups of 64) owns 64 channels:
// thread (g, lane) of channel lane reads inner-history rows g, g + 16, ...
// (each row once) into registers and adds its share of the inner FIR (HCS /
// HCM), or, for HCL, loads the pole, residue and state of modes 4g .. 4g+3
// (groups 0..3); group 0 forms the short FIR and gates of the projection
// row. After a barrier the history rows move one row down (the new u goes
// to the last row), group 1 shifts the short history, the HCL groups update
// their modes; the partial sums meet in LDS and group 0 finishes the
// channel (outer gate). Sums as in hyena_fir_kernel except that the history
// part is added per row group (groups 0..15 in order); the modal sum adds
// the four mode groups in order.
constexpr int kDecodeGroups = 16;
constexpr int kDecodeRowsPerThread = 8;  // ceil(127 / 16)

template <typename T, typename O>
__global__ __launch_bounds__(64 * kDecodeGroups) void hyena_decode_kernel(
    int kind, const T *__restrict__ P, float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len, float *__restrict__ inner_history,
    const float *__restrict__ filter, size_t groups, int k, int causal,
    const float *__restrict__ direct, const float *__restrict__ poles,
    const float *__restrict__ residues, float *__restrict__ modal_state, int S, size_t W,
    O out) {
  __shared__ float partial_s[kDecodeGroups][64];
  __shared__ float u_s[64];
  const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
  const size_t c = blockIdx.x * 64ULL + lane;
  const bool valid = c < W;
  const size_t cols3 = 3 * W;
  float x2 = 0.0F, u = 0.0F;
  if (g == 0 && valid) {
    float taps[3][kMaxShort];
    load_short_taps(short_filter, short_len, c, taps);
    gates(P, short_history, taps, short_len, cols3, 0, 0, c, &x2, &u);
    u_s[lane] = u;
  }
  const bool fir = kind != kHyenaHcl;
  const int hist = k - 1;
  float part = 0.0F;
  float v[kDecodeRowsPerThread];
  if (fir && valid && inner_history != nullptr) {
    const float *h = filter + (c / (W / groups)) * k;
#pragma unroll
    for (int i = 0; i < kDecodeRowsPerThread; ++i) {
      const int old = g + kDecodeGroups * i;
      v[i] = old < hist ? inner_history[old * W + c] : 0.0F;
    }
#pragma unroll
    for (int i = 0; i < kDecodeRowsPerThread; ++i) {
      const int old = g + kDecodeGroups * i;
      if (old < hist)
        part += v[i] * h[causal ? k - 1 - old : old];
    }
  }
  // HCL: modes 4g .. 4g+3 of the channel, loaded before the barrier.
  const bool modal = !fir && valid && g < 4;
  float pm[4] = {}, rm[4] = {}, st[4] = {};
  if (modal) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 4 * g + e;
      if (m < S) {
        pm[e] = poles[c * S + m];
        rm[e] = residues[c * S + m];
        st[e] = modal_state != nullptr ? modal_state[c * S + m] : 0.0F;
      }
    }
  }
  partial_s[g][lane] = part;
  __syncthreads();  // every history row read; u of the block's channels ready
  if (fir && valid && inner_history != nullptr) {
#pragma unroll
    for (int i = 0; i < kDecodeRowsPerThread; ++i) {
      const int old = g + kDecodeGroups * i;
      if (old >= 1 && old < hist)
        inner_history[(old - 1) * W + c] = v[i];
    }
    if (g == 0 && hist > 0)
      inner_history[(hist - 1) * W + c] = u_s[lane];
  }
  if (g == 1 && valid && short_history != nullptr && short_len > 1) {
    // Group 0 read the short history before the barrier.
    const int rows = short_len - 1;
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      const size_t col = 3 * c + s;
      for (int h = 0; h + 1 < rows; ++h)
        short_history[h * cols3 + col] = short_history[(h + 1) * cols3 + col];
      short_history[(rows - 1) * cols3 + col] = load_act(P, col);
    }
  }
  if (!fir) {
    if (modal) {
      const float uc = u_s[lane];
      float sum = 0.0F;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 4 * g + e;
        if (m < S) {
          st[e] = pm[e] * st[e] + uc;
          if (modal_state != nullptr)
            modal_state[c * S + m] = st[e];
          sum += rm[e] * st[e];
        }
      }
      partial_s[g][lane] = sum;
    }
    __syncthreads();  // the mode groups' sums
  }
  if (g != 0 || !valid)
    return;
  float total;
  if (!fir) {
    const float modal_sum =
        ((partial_s[0][lane] + partial_s[1][lane]) + partial_s[2][lane]) + partial_s[3][lane];
    total = modal_sum + direct[c] * u;
  } else {
    const float *h = filter + (c / (W / groups)) * k;
    total = 0.0F;
#pragma unroll
    for (int q = 0; q < kDecodeGroups; ++q)
      total += partial_s[q][lane];
    total += u * h[causal ? 0 : hist];
    if (direct != nullptr)
      total += direct[c] * u;
  }
  put(out, c, x2 * total);
}

size_t hcl_chunks(size_t length) { return (length + kChunk - 1) / kChunk; }

template <typename T, typename O, int kWin>
Status launch_hcl(const T *projection, const float *short_history, const HyenaWeights &wt,
                  int short_len, size_t length, size_t width, size_t planar, int S, size_t G,
                  float *chunk_state, float *modal_state, O out, hipStream_t stream) {
  const dim3 grid(ceil_div(width, kChannels), static_cast<unsigned>(G));
  hipLaunchKernelGGL((hcl_chunk_state_kernel<T, kWin>), grid, dim3(kChannels), 0, stream,
                     projection, short_history, wt.short_filter, short_len, length, width,
                     planar, wt.poles, S, chunk_state);
  EVO_TRY(launch_status("hcl_chunk_state_kernel"));
  hipLaunchKernelGGL(hcl_carry_kernel, dim3(ceil_div(width * S, 256)), dim3(256), 0, stream,
                     chunk_state, G, length, width, S, wt.poles, modal_state);
  EVO_TRY(launch_status("hcl_carry_kernel"));
  hipLaunchKernelGGL((hcl_output_kernel<T, O, kWin>), grid, dim3(kChannels), 0, stream,
                     projection, short_history, wt.short_filter, short_len, length, width,
                     planar, wt.poles, wt.residues, wt.direct, S, chunk_state, out);
  return launch_status("hcl_output_kernel");
}

template <typename T, typename O, int kWin, int kTaps>
void launch_fir_stream_taps(const T *projection, const float *short_history,
                            const HyenaWeights &wt, int short_len, const float *inner_history,
                            size_t group_size, int k, int causal, const float *direct,
                            size_t length, size_t width, O out, hipStream_t stream) {
  const unsigned cblocks = ceil_div(width, kStreamChannels);
  unsigned seg_len = kStreamRows;
  while (seg_len < kStreamMaxRows &&
         cblocks * ceil_div(length, 2 * static_cast<size_t>(seg_len)) >= kStreamMinBlocks)
    seg_len *= 2;
  const unsigned segments = ceil_div(length, seg_len);
  const dim3 grid(cblocks * segments), block(kStreamWaves * 64);
  if (direct != nullptr)
    hipLaunchKernelGGL((hyena_fir_stream_kernel<T, O, kWin, kTaps, true>), grid, block, 0, stream,
                       projection, short_history, wt.short_filter, short_len, inner_history,
                       wt.inner_filter, group_size, k, causal, direct, length, width, cblocks,
                       segments, seg_len, out);
  else
    hipLaunchKernelGGL((hyena_fir_stream_kernel<T, O, kWin, kTaps, false>), grid, block, 0,
                       stream, projection, short_history, wt.short_filter, short_len,
                       inner_history, wt.inner_filter, group_size, k, causal, direct, length,
                       width, cblocks, segments, seg_len, out);
}

// Exact window widths for the 7B shape (short FIR 3, HCS 7 taps); other
// lengths run zero-padded windows of 8.
template <typename T, typename O>
Status launch_fir_stream(const T *projection, const float *short_history,
                         const HyenaWeights &wt, int short_len, const float *inner_history,
                         size_t group_size, int k, int causal, const float *direct,
                         size_t length, size_t width, O out, hipStream_t stream) {
  if (short_len == 3 && k == 7)
    launch_fir_stream_taps<T, O, 3, 7>(projection, short_history, wt, short_len, inner_history,
                                       group_size, k, causal, direct, length, width, out, stream);
  else
    launch_fir_stream_taps<T, O, kMaxShort, 8>(projection, short_history, wt, short_len,
                                               inner_history, group_size, k, causal, direct,
                                               length, width, out, stream);
  return launch_status("hyena_fir_stream_kernel");
}

template <typename T, typename O, int kMaxTaps>
Status launch_fir_mfma(const T *projection, const float *short_history,
                       const HyenaWeights &wt, int short_len, const float *inner_history,
                       size_t group_size, int k, int causal, const float *direct,
                       size_t length, size_t width, size_t planar, void *workspace, O out,
                       hipStream_t stream) {
  constexpr size_t lds = FirMfmaShape<kMaxTaps>::kLdsBytes;
  static_assert(lds <= 160 * 1024, "LDS");
  auto *fragments = static_cast<uint4 *>(workspace);
  hipLaunchKernelGGL(toeplitz_fragments_kernel<kMaxTaps>,
                     dim3(static_cast<unsigned>(wt.groups), FirMfmaShape<kMaxTaps>::kSteps),
                     dim3(64), 0, stream, wt.inner_filter, k, causal, fragments);
  EVO_TRY(launch_status("toeplitz_fragments_kernel"));
  const dim3 grid(static_cast<unsigned>(width / kChannels),
                  static_cast<unsigned>(ceil_div(length, kFirTile)));
  if (short_len <= 4) {
    auto kernel = hyena_fir_mfma_kernel<T, O, kMaxTaps, 4>;
    EVO_TRY(hip_status(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(lds)),
                       "hyena_fir_mfma_kernel LDS opt-in"));
    hipLaunchKernelGGL(kernel, grid, dim3(kFirThreads), lds, stream, projection,
                       short_history, wt.short_filter, short_len, inner_history,
                       fragments, group_size, k, causal, direct, length, width, planar, out);
  } else {
    auto kernel = hyena_fir_mfma_kernel<T, O, kMaxTaps, kMaxShort>;
    EVO_TRY(hip_status(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(lds)),
                       "hyena_fir_mfma_kernel LDS opt-in"));
    hipLaunchKernelGGL(kernel, grid, dim3(kFirThreads), lds, stream, projection,
                       short_history, wt.short_filter, short_len, inner_history,
                       fragments, group_size, k, causal, direct, length, width, planar, out);
  }
  return launch_status("hyena_fir_mfma_kernel");
}

}  // namespace

size_t hyena_workspace_bytes(int kind, size_t length, size_t width,
                             size_t state) {
  if (kind == kHyenaHcs || kind == kHyenaHcm) {
    // Toeplitz fragment table of the MFMA FIR: at most width/16 groups of
    // kSteps x 2 planes x 64 lanes x 16 bytes.
    if (width % kChannels != 0)
      return 0;
    const size_t steps = kind == kHyenaHcs ? FirMfmaShape<8>::kSteps : FirMfmaShape<128>::kSteps;
    return width / 16 * steps * 2 * 64 * 16;
  }
  if (kind != kHyenaHcl)
    return 0;
  return hcl_chunks(length) * state * width * sizeof(float);
}

template <typename T, typename O>
Status hyena_forward(int kind, const T *projection, size_t length,
                     size_t width, bool planar_projection, const HyenaWeights &wt,
                     float *short_history, float *inner_history,
                     float *modal_state, void *workspace,
                     size_t workspace_bytes, O out, hipStream_t stream) {
  if (projection == nullptr || wt.short_filter == nullptr ||
      length == 0 || width == 0 || wt.short_len < 1 ||
      wt.short_len > kMaxShort || length > (1UL << 40))
    return {ErrorCode::kInvalidArgument, "hyena_forward: invalid arguments"};
  const int short_len = static_cast<int>(wt.short_len);
  const size_t planar = planar_projection ? width : 0;
  const dim3 channel_blocks(ceil_div(width, kChannels));
  // One row (decode): the whole operator and both history updates in one
  // launch.
  if (length == 1 && planar == 0 &&
      ((kind == kHyenaHcl && wt.poles != nullptr && wt.residues != nullptr &&
        wt.direct != nullptr && wt.state >= 1 && wt.state <= kMaxState) ||
       ((kind == kHyenaHcs || kind == kHyenaHcm) && wt.inner_filter != nullptr &&
        wt.groups != 0 && width % wt.groups == 0 && wt.inner_len >= 1 &&
        wt.inner_len <= 128 && (kind == kHyenaHcs || wt.direct != nullptr)))) {
    const bool hcm = kind == kHyenaHcm;
    hipLaunchKernelGGL((hyena_decode_kernel<T, O>), dim3(ceil_div(width, 64)),
                       dim3(64 * kDecodeGroups), 0,
                       stream, kind, projection, short_history, wt.short_filter, short_len,
                       inner_history, wt.inner_filter, wt.groups,
                       static_cast<int>(wt.inner_len), hcm ? 1 : 0,
                       kind == kHyenaHcs ? nullptr : wt.direct, wt.poles, wt.residues,
                       modal_state, static_cast<int>(wt.state), width, out);
    return launch_status("hyena_decode_kernel");
  }
  if (kind == kHyenaHcl) {
    if (wt.poles == nullptr || wt.residues == nullptr || wt.direct == nullptr ||
        wt.state == 0 || wt.state > kMaxState)
      return {ErrorCode::kInvalidArgument, "hyena_forward: HCL needs poles, residues, D, 1..16 states"};
    if (short_len == 3 && planar == 0 && width % kHmChannels == 0) {
      // One pass on MFMA; the modal state stays in the block (no workspace).
      const unsigned blocks = static_cast<unsigned>(width / kHmChannels);
      hipLaunchKernelGGL((hcl_mfma_kernel<T, O>), dim3(blocks), dim3(kHmThreads<O>), 0, stream,
                         projection, short_history, wt.short_filter, length, width, wt.poles,
                         wt.residues, wt.direct, static_cast<int>(wt.state), modal_state, out);
      EVO_TRY(launch_status("hcl_mfma_kernel"));
      if (short_history != nullptr) {
        hipLaunchKernelGGL(short_history_kernel<T>, dim3(ceil_div(3 * width, 256)), dim3(256),
                           0, stream, projection, length, 3 * width, short_history,
                           short_len - 1);
        EVO_TRY(launch_status("short_history_kernel"));
      }
      return Status::Ok();
    }
    const size_t G = hcl_chunks(length);
    if (workspace == nullptr ||
        workspace_bytes < hyena_workspace_bytes(kind, length, width, wt.state))
      return {ErrorCode::kInvalidArgument, "hyena_forward: HCL workspace too small"};
    if (G > 65535)
      return {ErrorCode::kInvalidArgument, "hyena_forward: sequence too long for one call"};
    float *chunk_state = static_cast<float *>(workspace);
    const int S = static_cast<int>(wt.state);
    if (short_len == 3 && planar == 0 && width % 2 == 0) {
      const dim3 grid(ceil_div(width, 256), static_cast<unsigned>(G));
      hipLaunchKernelGGL(hcl_state_pair_kernel<T>, grid, dim3(256), 0, stream, projection,
                         short_history, wt.short_filter, length, width, wt.poles, S,
                         chunk_state);
      EVO_TRY(launch_status("hcl_state_pair_kernel"));
      hipLaunchKernelGGL(hcl_carry_seg_kernel, dim3(ceil_div(width, 64), S), dim3(256), 0,
                         stream, chunk_state, G, length, width, S, wt.poles, modal_state);
      EVO_TRY(launch_status("hcl_carry_seg_kernel"));
      hipLaunchKernelGGL((hcl_output_pair_kernel<T, O>), grid, dim3(256), 0, stream,
                         projection, short_history, wt.short_filter, length, width, wt.poles,
                         wt.residues, wt.direct, S, chunk_state, out);
      EVO_TRY(launch_status("hcl_output_pair_kernel"));
    } else if (short_len <= 4) {
      EVO_TRY((launch_hcl<T, O, 4>(projection, short_history, wt, short_len, length, width,
                                   planar, S, G, chunk_state, modal_state, out, stream)));
    } else {
      EVO_TRY((launch_hcl<T, O, kMaxShort>(projection, short_history, wt, short_len, length,
                                           width, planar, S, G, chunk_state, modal_state, out, stream)));
    }
  } else if (kind == kHyenaHcs || kind == kHyenaHcm) {
    if (wt.inner_filter == nullptr || wt.groups == 0 || width % wt.groups != 0 ||
        wt.inner_len < 1 || wt.inner_len > 128 ||
        (kind == kHyenaHcm && wt.direct == nullptr))
      return {ErrorCode::kInvalidArgument, "hyena_forward: FIR needs taps (<=128), groups dividing W"};
    const int k = static_cast<int>(wt.inner_len);
    const int causal = kind == kHyenaHcm ? 1 : 0;
    const float *direct = kind == kHyenaHcm ? wt.direct : nullptr;
    const size_t group_size = width / wt.groups;
    if (k <= 8 && planar == 0 && width % 2 == 0 && group_size % 2 == 0) {
      EVO_TRY((launch_fir_stream<T, O>(projection, short_history, wt, short_len, inner_history,
                                       group_size, k, causal, direct, length, width, out,
                                       stream)));
    } else if (wt.taps_bf16 && short_len == 3 && planar == 0 && width % kMsChannels == 0 &&
               group_size % 16 == 0 && direct != nullptr) {
      const unsigned cblocks = static_cast<unsigned>(width / kMsChannels);
      unsigned seg_len = kMsSegment;
      while (seg_len > kMsMinSegment && cblocks * ceil_div(length, seg_len) < kMsMinBlocks)
        seg_len /= 2;
      const unsigned segments = ceil_div(length, seg_len);
      hipLaunchKernelGGL((hyena_fir_mfma_stream_kernel<T, O>), dim3(cblocks * segments),
                         dim3(256), 0, stream, projection, short_history, wt.short_filter,
                         short_len, inner_history, wt.inner_filter, group_size, k, causal, direct,
                         length, width, cblocks, segments, seg_len, out);
      EVO_TRY(launch_status("hyena_fir_mfma_stream_kernel"));
    } else if (width % kChannels == 0 && group_size % 16 == 0) {
      const size_t steps = k <= 8 ? FirMfmaShape<8>::kSteps : FirMfmaShape<128>::kSteps;
      if (workspace == nullptr || workspace_bytes < wt.groups * steps * 2 * 64 * 16)
        return {ErrorCode::kInvalidArgument, "hyena_forward: FIR workspace too small"};
      if (k <= 8) {
        EVO_TRY((launch_fir_mfma<T, O, 8>(projection, short_history, wt, short_len,
                                          inner_history, group_size, k, causal, direct, length,
                                          width, planar, workspace, out, stream)));
      } else {
        EVO_TRY((launch_fir_mfma<T, O, 128>(projection, short_history, wt, short_len,
                                            inner_history, group_size, k, causal, direct,
                                            length, width, planar, workspace, out, stream)));
      }
    } else if (k <= 8) {
      constexpr int kTile = 64, kTaps = 8;
      static_assert(((kTaps - 1 + kTile) + kTile) * 64 * sizeof(float) <= 65536, "LDS");
      const size_t lds = ((kTaps - 1 + kTile) + kTile) * 64 * sizeof(float);
      const dim3 grid(channel_blocks.x, ceil_div(length, kTile));
      hipLaunchKernelGGL((hyena_fir_kernel<T, O, kTile, kTaps>), grid, dim3(256), lds, stream,
                         projection, short_history, wt.short_filter, short_len,
                         inner_history, wt.inner_filter, wt.groups, k, causal,
                         direct, length, width, planar, out);
    } else {
      constexpr int kTile = 128, kTaps = 128;
      const size_t lds = ((kTaps - 1 + kTile) + kTile) * 64 * sizeof(float);
      // 98 KB of the CU's 160 KB LDS: opt in above the 64 KB default.
      EVO_TRY(hip_status(hipFuncSetAttribute(
                             reinterpret_cast<const void *>(&hyena_fir_kernel<T, O, kTile, kTaps>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
                         "hyena_fir_kernel LDS opt-in"));
      const dim3 grid(channel_blocks.x, ceil_div(length, kTile));
      hipLaunchKernelGGL((hyena_fir_kernel<T, O, kTile, kTaps>), grid, dim3(256), lds, stream,
                         projection, short_history, wt.short_filter, short_len,
                         inner_history, wt.inner_filter, wt.groups, k, causal,
                         direct, length, width, planar, out);
    }
    EVO_TRY(launch_status("hyena_fir_kernel"));
    if (inner_history != nullptr && k > 1) {
      if (length >= static_cast<size_t>(k - 1)) {
        hipLaunchKernelGGL(inner_history_kernel<T>, dim3(ceil_div(width, 256), k - 1),
                           dim3(256), 0, stream, projection, short_history, wt.short_filter,
                           short_len, length, width, planar, inner_history, k - 1);
      } else {
        const size_t lds = static_cast<size_t>(k - 1) * 64 * sizeof(float);  // <= 32.5 KB
        hipLaunchKernelGGL(inner_history_shift_kernel<T>, dim3(ceil_div(width, 64)), dim3(256),
                           lds, stream, projection, short_history, wt.short_filter, short_len,
                           length, width, planar, inner_history, k - 1);
      }
      EVO_TRY(launch_status("inner_history_kernel"));
    }
  } else {
    return {ErrorCode::kInvalidArgument, "hyena_forward: unknown kind"};
  }
  if (short_history != nullptr && short_len > 1) {
    hipLaunchKernelGGL(short_history_kernel<T>, dim3(ceil_div(3 * width, 256)), dim3(256), 0,
                       stream, projection, length, 3 * width, short_history,
                       short_len - 1);
    EVO_TRY(launch_status("short_history_kernel"));
  }
  return Status::Ok();
}

template Status hyena_forward<float, float *>(int, const float *, size_t, size_t, bool,
                                              const HyenaWeights &, float *, float *,
                                              float *, void *, size_t, float *,
                                              hipStream_t);
template Status hyena_forward<uint16_t, uint16_t *>(int, const uint16_t *, size_t, size_t, bool,
                                                    const HyenaWeights &, float *, float *,
                                                    float *, void *, size_t, uint16_t *,
                                                    hipStream_t);
template Status hyena_forward<uint16_t, SplitOut>(int, const uint16_t *, size_t, size_t, bool,
                                                  const HyenaWeights &, float *, float *,
                                                  float *, void *, size_t, SplitOut,
                                                  hipStream_t);
template Status hyena_forward<float, SplitOut>(int, const float *, size_t, size_t, bool,
                                               const HyenaWeights &, float *, float *,
                                               float *, void *, size_t, SplitOut,
                                               hipStream_t);
template Status hyena_forward<uint16_t, F16Out>(int, const uint16_t *, size_t, size_t, bool,
                                                const HyenaWeights &, float *, float *,
                                                float *, void *, size_t, F16Out,
                                                hipStream_t);
template Status hyena_forward<float, F16Out>(int, const float *, size_t, size_t, bool,
                                             const HyenaWeights &, float *, float *,
                                             float *, void *, size_t, F16Out,
                                             hipStream_t);

// ---- Fixed scratch of the allocation-free operator entry point.
// One array per device, alive until the process ends. Its host-side name is
// not a device address: host code only ever uses the address that
// hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[kHyenaStaticScratchBytes];

Status hyena_static_scratch(void **address) {
  constexpr int kMaxDevices = 64;
  static std::mutex mutex;
  static void *per_device[kMaxDevices] = {};
  int device = 0;
  EVO_TRY(hip_status(hipGetDevice(&device), "hyena static scratch: current device"));
  if (device < 0 || device >= kMaxDevices)
    return {ErrorCode::kInvalidArgument, "hyena static scratch: device index out of range"};
  std::lock_guard<std::mutex> lock(mutex);
  if (per_device[device] == nullptr) {
    void *ptr = nullptr;
    EVO_TRY(hip_status(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)),
                       "hyena static scratch: symbol address"));
    per_device[device] = ptr;
  }
  *address = per_device[device];
  return Status::Ok();
}

}  // namespace evo::hip
