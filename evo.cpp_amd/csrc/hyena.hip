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

namespace evo::hip {
namespace {

constexpr int kChannels = 64;    // channels per block (one wave)
constexpr int kChunk = 64;       // HCL rows per chunk
constexpr int kMaxState = 16;
constexpr int kMaxShort = 8;

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
                             size_t cols3, long t, size_t c, float *x2,
                             float *u) {
  *x2 = short_fir(P, short_history, taps[0], k, cols3, t, 3 * c);
  const float x1 = short_fir(P, short_history, taps[1], k, cols3, t, 3 * c + 1);
  const float v = short_fir(P, short_history, taps[2], k, cols3, t, 3 * c + 2);
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
                        size_t cols3, long t0, size_t c) {
#pragma unroll
    for (int i = 0; i < kWin - 1; ++i) {
      const long t = t0 - (kWin - 1) + i;
      // Rows older than the filter reach only meet zero taps.
      const bool used = t >= t0 - (k - 1);
#pragma unroll
      for (int s = 0; s < 3; ++s)
        win[s][i + 1] = used ? p_at(P, short_history, cols3, k - 1, t, 3 * c + s) : 0.0F;
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

// Loads rows [t, t + kBatch) (clipped to t1) of the channel's 3 columns.
template <typename T>
__device__ inline void load_batch(const T *P, size_t cols3, size_t t, size_t t1,
                                  size_t c, float (&rows)[kBatch][3]) {
#pragma unroll
  for (int b = 0; b < kBatch; ++b)
#pragma unroll
    for (int s = 0; s < 3; ++s)
      rows[b][s] = t + b < t1 ? load_act(P, (t + b) * cols3 + 3 * c + s) : 0.0F;
}

// ---- HCL phase 1: final local state of every chunk from a zero start.
template <typename T, int kWin>
__global__ __launch_bounds__(kChannels) void hcl_chunk_state_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len, size_t L,
    size_t W, const float *__restrict__ poles, int S, float *__restrict__ chunk_state) {
  const size_t c = blockIdx.x * static_cast<size_t>(kChannels) + threadIdx.x;
  if (c >= W)
    return;
  const size_t g = blockIdx.y;
  const size_t t0 = g * kChunk, t1 = min(L, t0 + kChunk);
  const size_t cols3 = 3 * W;
  RowStream<T, kWin> stream;
  load_window_taps(short_filter, short_len, c, stream.taps);
  stream.prime(P, short_history, short_len, cols3, static_cast<long>(t0), c);
  float p[kMaxState], s[kMaxState];
#pragma unroll
  for (int m = 0; m < kMaxState; ++m) {
    p[m] = m < S ? poles[c * S + m] : 0.0F;
    s[m] = 0.0F;
  }
  for (size_t t = t0; t < t1; t += kBatch) {
    float rows[kBatch][3];
    load_batch(P, cols3, t, t1, c, rows);
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
  for (size_t g = 0; g < G; ++g) {
    const size_t index = (g * S + m) * W + c;
    const float local = chunk_state[index];
    chunk_state[index] = state;
    const size_t len = min(L - g * kChunk, static_cast<size_t>(kChunk));
    float power = full;
    if (len != static_cast<size_t>(kChunk)) {
      power = 1.0F;
      for (size_t e = 0; e < len; ++e)
        power *= p;
    }
    state = power * state + local;
  }
  if (modal_state != nullptr)
    modal_state[c * S + m] = state;
}

// ---- HCL phase 3: rescan each chunk from its true start state.
template <typename T, typename O, int kWin>
__global__ __launch_bounds__(kChannels) void hcl_output_kernel(
    const T *__restrict__ P, const float *__restrict__ short_history,
    const uint16_t *__restrict__ short_filter, int short_len, size_t L,
    size_t W, const float *__restrict__ poles,
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
  stream.prime(P, short_history, short_len, cols3, static_cast<long>(t0), c);
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
    load_batch(P, cols3, t, t1, c, rows);
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
      put(out, (t + b) * W + c, x2 * (modal + d * u));
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
    size_t L, size_t W, O out) {
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
        gates(P, short_history, taps, short_len, cols3, t, c, &x2, &u);
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

// Rewrites the inner (u) history with the last k-1 rows of [history ; u].
// Runs after the main kernel and before the short history moves on.
template <typename T>
__global__ void inner_history_kernel(const T *__restrict__ P,
                                     const float *__restrict__ short_history,
                                     const uint16_t *__restrict__ short_filter,
                                     int short_len, size_t L, size_t W,
                                     float *inner_history, int hist) {
  const size_t c = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (c >= W)
    return;
  float taps[3][kMaxShort];
  load_short_taps(short_filter, short_len, c, taps);
  const size_t cols3 = 3 * W;
  for (int h = 0; h < hist; ++h) {
    const long source = static_cast<long>(h) + static_cast<long>(L);  // in [hist ; u]
    float value;
    if (source < hist) {
      value = inner_history[static_cast<size_t>(source) * W + c];
    } else {
      const long t = source - hist;
      float x2, u;
      gates(P, short_history, taps, short_len, cols3, t, c, &x2, &u);
      value = u;
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

size_t hcl_chunks(size_t length) { return (length + kChunk - 1) / kChunk; }

template <typename T, typename O, int kWin>
Status launch_hcl(const T *projection, const float *short_history, const HyenaWeights &wt,
                  int short_len, size_t length, size_t width, int S, size_t G,
                  float *chunk_state, float *modal_state, O out, hipStream_t stream) {
  const dim3 grid(ceil_div(width, kChannels), static_cast<unsigned>(G));
  hipLaunchKernelGGL((hcl_chunk_state_kernel<T, kWin>), grid, dim3(kChannels), 0, stream,
                     projection, short_history, wt.short_filter, short_len, length, width,
                     wt.poles, S, chunk_state);
  EVO_TRY(launch_status("hcl_chunk_state_kernel"));
  hipLaunchKernelGGL(hcl_carry_kernel, dim3(ceil_div(width * S, 256)), dim3(256), 0, stream,
                     chunk_state, G, length, width, S, wt.poles, modal_state);
  EVO_TRY(launch_status("hcl_carry_kernel"));
  hipLaunchKernelGGL((hcl_output_kernel<T, O, kWin>), grid, dim3(kChannels), 0, stream,
                     projection, short_history, wt.short_filter, short_len, length, width,
                     wt.poles, wt.residues, wt.direct, S, chunk_state, out);
  return launch_status("hcl_output_kernel");
}

}  // namespace

size_t hyena_workspace_bytes(int kind, size_t length, size_t width,
                             size_t state) {
  if (kind != kHyenaHcl)
    return 0;
  return hcl_chunks(length) * state * width * sizeof(float);
}

template <typename T, typename O>
Status hyena_forward(int kind, const T *projection, size_t length,
                     size_t width, const HyenaWeights &wt,
                     float *short_history, float *inner_history,
                     float *modal_state, void *workspace,
                     size_t workspace_bytes, O out, hipStream_t stream) {
  if (projection == nullptr || wt.short_filter == nullptr ||
      length == 0 || width == 0 || wt.short_len < 1 ||
      wt.short_len > kMaxShort || length > (1UL << 40))
    return {ErrorCode::kInvalidArgument, "hyena_forward: invalid arguments"};
  const int short_len = static_cast<int>(wt.short_len);
  const dim3 channel_blocks(ceil_div(width, kChannels));
  if (kind == kHyenaHcl) {
    if (wt.poles == nullptr || wt.residues == nullptr || wt.direct == nullptr ||
        wt.state == 0 || wt.state > kMaxState)
      return {ErrorCode::kInvalidArgument, "hyena_forward: HCL needs poles, residues, D, 1..16 states"};
    const size_t G = hcl_chunks(length);
    if (workspace == nullptr ||
        workspace_bytes < hyena_workspace_bytes(kind, length, width, wt.state))
      return {ErrorCode::kInvalidArgument, "hyena_forward: HCL workspace too small"};
    if (G > 65535)
      return {ErrorCode::kInvalidArgument, "hyena_forward: sequence too long for one call"};
    float *chunk_state = static_cast<float *>(workspace);
    const int S = static_cast<int>(wt.state);
    if (short_len <= 4) {
      EVO_TRY((launch_hcl<T, O, 4>(projection, short_history, wt, short_len, length, width,
                                   S, G, chunk_state, modal_state, out, stream)));
    } else {
      EVO_TRY((launch_hcl<T, O, kMaxShort>(projection, short_history, wt, short_len, length,
                                           width, S, G, chunk_state, modal_state, out, stream)));
    }
  } else if (kind == kHyenaHcs || kind == kHyenaHcm) {
    if (wt.inner_filter == nullptr || wt.groups == 0 || width % wt.groups != 0 ||
        wt.inner_len < 1 || wt.inner_len > 128 ||
        (kind == kHyenaHcm && wt.direct == nullptr))
      return {ErrorCode::kInvalidArgument, "hyena_forward: FIR needs taps (<=128), groups dividing W"};
    const int k = static_cast<int>(wt.inner_len);
    const int causal = kind == kHyenaHcm ? 1 : 0;
    const float *direct = kind == kHyenaHcm ? wt.direct : nullptr;
    if (k <= 8) {
      constexpr int kTile = 64, kTaps = 8;
      static_assert(((kTaps - 1 + kTile) + kTile) * 64 * sizeof(float) <= 65536, "LDS");
      const size_t lds = ((kTaps - 1 + kTile) + kTile) * 64 * sizeof(float);
      const dim3 grid(channel_blocks.x, ceil_div(length, kTile));
      hipLaunchKernelGGL((hyena_fir_kernel<T, O, kTile, kTaps>), grid, dim3(256), lds, stream,
                         projection, short_history, wt.short_filter, short_len,
                         inner_history, wt.inner_filter, wt.groups, k, causal,
                         direct, length, width, out);
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
                         direct, length, width, out);
    }
    EVO_TRY(launch_status("hyena_fir_kernel"));
    if (inner_history != nullptr && k > 1) {
      hipLaunchKernelGGL(inner_history_kernel<T>, dim3(ceil_div(width, 256)), dim3(256), 0,
                         stream, projection, short_history, wt.short_filter,
                         short_len, length, width, inner_history, k - 1);
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

template Status hyena_forward<float, float *>(int, const float *, size_t, size_t,
                                              const HyenaWeights &, float *, float *,
                                              float *, void *, size_t, float *,
                                              hipStream_t);
template Status hyena_forward<uint16_t, uint16_t *>(int, const uint16_t *, size_t, size_t,
                                                    const HyenaWeights &, float *, float *,
                                                    float *, void *, size_t, uint16_t *,
                                                    hipStream_t);
template Status hyena_forward<uint16_t, SplitOut>(int, const uint16_t *, size_t, size_t,
                                                  const HyenaWeights &, float *, float *,
                                                  float *, void *, size_t, SplitOut,
                                                  hipStream_t);
template Status hyena_forward<float, SplitOut>(int, const float *, size_t, size_t,
                                               const HyenaWeights &, float *, float *,
                                               float *, void *, size_t, SplitOut,
                                               hipStream_t);

}  // namespace evo::hip
