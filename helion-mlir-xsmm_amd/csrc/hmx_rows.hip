// Memory-bound row kernels for gfx950: softmax, RMSNorm, GroupNorm/LayerNorm,
// row sums, row dots, gemv, column sums and elementwise ops.
//
// A row (or one (row, group) unit) is read once from HBM with 16-byte loads
// (`global_load_dwordx4`) into registers, reduced, and written once with
// non-temporal stores: one HBM read and one write per element, the floor for
// these ops. Rows of at most 64 vectors take the smallest power-of-two group
// of lanes that holds them (several rows per wave), rows of up to 128
// vectors one wave each (four rows per 256-thread workgroup). Longer rows take a whole
// workgroup of WPR waves (up to 16) holding two or more vectors per lane and
// combine the per-wave reductions through LDS: a [32768, 4096] f32 softmax
// runs 32768 workgroups of 8 waves with 8 values per lane, which measures
// ~25% more bandwidth on gfx950 than one wave holding the 4096-value row (64
// values per lane, 5 waves per SIMD). Rows longer than the register cache
// (16 waves x 64 values per lane) stream through the same math in chunks, one
// wave per row.
#include <atomic>
#include <type_traits>
#include <utility>

#include "hmx_rows_common.hpp"

namespace hmx {
namespace {

// ---------------------------------------------------------------------------
// Softmax: max, sum of exp(x - max), then exp(x - max) * (1 / sum), as
// helion_mlir_utils/normalization.py:47-72 computes it (f32 inside, one
// rounding), with the row held in registers between the passes. The grid
// holds exactly the rows (tpr > 64: one workgroup per row), so no thread that
// reaches a barrier has returned early.
template <typename T, int EPV, int VPL, bool WHOLE>
__global__ __launch_bounds__(kMaxBlock) void softmax_cached(const T* x, T* y, int64_t m,
                                                            int64_t n, int tpr) {
  __shared__ float red_max[kMaxWavesPerRow], red_sum[kMaxWavesPerRow];
  const RowPos p = row_pos(tpr);
  if (p.row >= m) return;
  float v[VPL * EPV];
  load_row<T, EPV, VPL, WHOLE>(x + p.row * n, n, p.li, p.tpr, v, -INFINITY);
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < VPL * EPV; ++i) mx = fmaxf(mx, v[i]);
  mx = row_max_all(mx, red_max, tpr);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < VPL * EPV; ++i) {
    v[i] = exp_sub(v[i], mx);
    if (WHOLE || col_of<EPV>(i / EPV, p.li, p.tpr, i % EPV) < n) sum += v[i];
  }
  sum = row_sum_all(sum, red_sum, tpr);
  const float inv = 1.f / sum;
#pragma unroll
  for (int i = 0; i < VPL * EPV; ++i) v[i] *= inv;
  store_row<T, EPV, VPL, WHOLE>(y + p.row * n, n, p.li, p.tpr, v);
}

template <typename T, int EPV>
__global__ __launch_bounds__(kBlock) void softmax_stream(const T* x,
                                                         T* y, int64_t m,
                                                         int64_t n) {
  const int64_t row = unit_index();
  if (row >= m) return;
  const int lane = threadIdx.x & (kWave - 1);
  const T* xr = x + row * n;
  T* yr = y + row * n;
  const int64_t step = (int64_t)kWave * EPV;
  float v[EPV];
  float mx = -INFINITY;
  for (int64_t col = (int64_t)lane * EPV; col < n; col += step) {
    load_chunk<T, EPV>(xr, n, col, v, -INFINITY);
#pragma unroll
    for (int e = 0; e < EPV; ++e) mx = fmaxf(mx, v[e]);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int64_t col = (int64_t)lane * EPV; col < n; col += step) {
    load_chunk<T, EPV>(xr, n, col, v, -INFINITY);
#pragma unroll
    for (int e = 0; e < EPV; ++e)
      if (col + e < n) sum += exp_sub(v[e], mx);
  }
  const float inv = 1.f / wave_sum(sum);
  for (int64_t col = (int64_t)lane * EPV; col < n; col += step) {
    load_chunk<T, EPV>(xr, n, col, v, 0.f);
#pragma unroll
    for (int e = 0; e < EPV; ++e) v[e] = exp_sub(v[e], mx) * inv;
    store_chunk<T, EPV>(yr, n, col, v);
  }
}

// ---------------------------------------------------------------------------
// RMSNorm: x * rsqrt(mean(x^2) + eps) * w in f32, rounded once. The weight
// (storage type W; null for none) is read with the same per-thread column map
// as x, so its loads are vectors too.
template <typename T, typename W, int EPV, int VPL, bool WHOLE>
__global__ __launch_bounds__(kMaxBlock) void rmsnorm_cached(const T* x, const W* __restrict__ w,
                                                            bool w_vec, T* y, int64_t m,
                                                            int64_t n, float eps, int tpr) {
  __shared__ float red_sum[kMaxWavesPerRow];
  const RowPos p = row_pos(tpr);
  if (p.row >= m) return;
  float v[VPL * EPV];
  load_row<T, EPV, VPL, WHOLE>(x + p.row * n, n, p.li, p.tpr, v, 0.f);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL * EPV; ++i) ss = __builtin_fmaf(v[i], v[i], ss);
  ss = row_sum_all(ss, red_sum, tpr);
  const float r = rsqrtf(ss / (float)n + eps);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    float wv[EPV];
    if (w != nullptr) {
      load_vec_run<W, EPV>(w, n, col_of<EPV>(j, p.li, p.tpr, 0), w_vec, wv);
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e) wv[e] = 1.f;
    }
#pragma unroll
    for (int e = 0; e < EPV; ++e) v[j * EPV + e] = v[j * EPV + e] * r * wv[e];
  }
  store_row<T, EPV, VPL, WHOLE>(y + p.row * n, n, p.li, p.tpr, v);
}

// RMSNorm of two rows per workgroup (rows of more than 64 threads, one row
// per workgroup in rmsnorm_cached; launched for bf16 rows): both rows' loads
// are in flight together and the weight is loaded once for the two. Each row's sum is the same as
// rmsnorm_cached's (same lanes, same order), so the results are equal.
template <typename T, typename W, int EPV, int VPL, bool WHOLE>
__global__ __launch_bounds__(kMaxBlock) void rmsnorm_cached2(const T* x, const W* __restrict__ w,
                                                             bool w_vec, T* y, int64_t m,
                                                             int64_t n, float eps, int tpr) {
  __shared__ float red_sum[2][kMaxWavesPerRow];
  const int li = (int)threadIdx.x;  // tpr == blockDim.x
  const int64_t r0 = (int64_t)blockIdx.x * 2;
  const bool two = r0 + 1 < m;
  float v0[VPL * EPV], v1[VPL * EPV];
  load_row<T, EPV, VPL, WHOLE>(x + r0 * n, n, li, tpr, v0, 0.f);
  if (two) {
    load_row<T, EPV, VPL, WHOLE>(x + (r0 + 1) * n, n, li, tpr, v1, 0.f);
  } else {
#pragma unroll
    for (int i = 0; i < VPL * EPV; ++i) v1[i] = 0.f;
  }
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = 0; i < VPL * EPV; ++i) {
    s0 = __builtin_fmaf(v0[i], v0[i], s0);
    s1 = __builtin_fmaf(v1[i], v1[i], s1);
  }
  s0 = row_sum_all(s0, red_sum[0], tpr);
  s1 = row_sum_all(s1, red_sum[1], tpr);
  const float q0 = rsqrtf(s0 / (float)n + eps), q1 = rsqrtf(s1 / (float)n + eps);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    float wv[EPV];
    if (w != nullptr) {
      load_vec_run<W, EPV>(w, n, col_of<EPV>(j, li, tpr, 0), w_vec, wv);
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e) wv[e] = 1.f;
    }
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      v0[j * EPV + e] = v0[j * EPV + e] * q0 * wv[e];
      v1[j * EPV + e] = v1[j * EPV + e] * q1 * wv[e];
    }
  }
  store_row<T, EPV, VPL, WHOLE>(y + r0 * n, n, li, tpr, v0);
  if (two) store_row<T, EPV, VPL, WHOLE>(y + (r0 + 1) * n, n, li, tpr, v1);
}

template <typename T, typename W, int EPV>
__global__ __launch_bounds__(kBlock) void rmsnorm_stream(const T* x, const W* __restrict__ w,
                                                         bool w_vec, T* y, int64_t m,
                                                         int64_t n, float eps) {
  const int64_t row = unit_index();
  if (row >= m) return;
  const int lane = threadIdx.x & (kWave - 1);
  const T* xr = x + row * n;
  T* yr = y + row * n;
  const int64_t step = (int64_t)kWave * EPV;
  float v[EPV];
  float ss = 0.f;
  for (int64_t col = (int64_t)lane * EPV; col < n; col += step) {
    load_chunk<T, EPV>(xr, n, col, v, 0.f);
#pragma unroll
    for (int e = 0; e < EPV; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
  }
  const float r = rsqrtf(wave_sum(ss) / (float)n + eps);
  for (int64_t col = (int64_t)lane * EPV; col < n; col += step) {
    load_chunk<T, EPV>(xr, n, col, v, 0.f);
    float wv[EPV];
    if (w != nullptr) {
      load_vec_run<W, EPV>(w, n, col, w_vec, wv);
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e) wv[e] = 1.f;
    }
#pragma unroll
    for (int e = 0; e < EPV; ++e) v[e] = v[e] * r * wv[e];
    store_chunk<T, EPV>(yr, n, col, v);
  }
}

// The value of channel ch before the activation: the normalized value, the
// extra op applied; with a program, the normalized value and (in `extra`)
// the extra operand the program reads.
__device__ __forceinline__ float group_norm_pre(const GroupNormArgs& a, float centered, float r,
                                                int64_t ch, float& extra) {
  float yv = centered * r * (a.w ? load_any(a.w, a.vec_dtype, ch) : 1.f);
  if (a.b) yv += load_any(a.b, a.vec_dtype, ch);
  extra = 0.f;
  if (a.act == HMX_EPI_PROGRAM) {
    if (a.extra) extra = load_any(a.extra, a.vec_dtype, ch);
    return yv;
  }
  if (a.extra_op == HMX_EXTRA_ADD) yv += load_any(a.extra, a.vec_dtype, ch);
  if (a.extra_op == HMX_EXTRA_MUL) yv *= load_any(a.extra, a.vec_dtype, ch);
  return yv;
}

template <typename T, int EPV, int VPL, bool WHOLE>
__global__ __launch_bounds__(kMaxBlock) void group_norm_cached(const T* x, T* y, GroupNormArgs a,
                                                               int tpr) {
  __shared__ float red_mean[kMaxWavesPerRow], red_var[kMaxWavesPerRow];
  const RowPos p = row_pos(tpr);
  const int64_t unit = p.row;
  if (unit >= a.units) return;
  const int64_t g = unit % a.groups;
  const int64_t n = a.gs;
  float v[VPL * EPV];
  load_row<T, EPV, VPL, WHOLE>(x + unit * n, n, p.li, p.tpr, v, 0.f);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL * EPV; ++i) s += v[i];
  const float mean = row_sum_all(s, red_mean, tpr) / (float)n;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VPL * EPV; ++i) {
    const float c = v[i] - mean;
    if (WHOLE || col_of<EPV>(i / EPV, p.li, p.tpr, i % EPV) < n) q += c * c;
  }
  const float r = rsqrtf(row_sum_all(q, red_var, tpr) / (float)n + a.eps);
  const bool prog = a.act == HMX_EPI_PROGRAM;
  float ex[VPL * EPV];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    if constexpr (EPV > 1) {
      const int64_t col0 = col_of<EPV>(j, p.li, p.tpr, 0);
      if (a.vec_ok && (WHOLE || col0 + EPV <= n)) {
        // The same arithmetic as group_norm_pre, on whole vectors of w, b, extra.
        float wv[EPV], bv[EPV], ev[EPV];
        load_vec_any<EPV>(a.w, a.vec_dtype, g * n + col0, wv, 1.f);
        load_vec_any<EPV>(a.b, a.vec_dtype, g * n + col0, bv, 0.f);
        load_vec_any<EPV>(a.extra_op != HMX_EXTRA_NONE || prog ? a.extra : nullptr, a.vec_dtype, g * n + col0,
                          ev, 0.f);
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          float yv = (v[j * EPV + e] - mean) * r * wv[e];
          yv += bv[e];
          if (!prog && a.extra_op == HMX_EXTRA_ADD) yv += ev[e];
          if (!prog && a.extra_op == HMX_EXTRA_MUL) yv *= ev[e];
          v[j * EPV + e] = yv;
          ex[j * EPV + e] = ev[e];
        }
        continue;
      }
    }
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const int64_t col = col_of<EPV>(j, p.li, p.tpr, e);
      ex[j * EPV + e] = 0.f;
      if (WHOLE || col < n)
        v[j * EPV + e] = group_norm_pre(a, v[j * EPV + e] - mean, r, g * n + col, ex[j * EPV + e]);
    }
  }
  group_norm_finish<VPL * EPV, false>(a, v, ex);
  store_row<T, EPV, VPL, WHOLE>(y + unit * n, n, p.li, p.tpr, v);
}

// Whole-row GroupNorm (body in hmx_rows_common.hpp). PROG: the epilogue is
// a program, run by the interpreter.
template <typename T, int EPV, int VPL, bool ONE, bool EXTRA, bool PROG = false>
__global__ __launch_bounds__(PROG ? kProgBlock : kMaxBlock) void group_norm_rows(const T* x, T* y, GroupNormArgs a,
                                                             int64_t rows, int tpr, int gv) {
  group_norm_rows_body<T, EPV, VPL, ONE, EXTRA, PROG ? EPI_PROGRAM : EPI_NAMED>(x, y, a, rows, tpr, gv);
}

template <typename T, int EPV, bool PROG>
__global__ __launch_bounds__(kBlock) void group_norm_stream(const T* x,
                                                            T* y,
                                                            GroupNormArgs a) {
  const int64_t unit = unit_index();
  if (unit >= a.units) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t g = unit % a.groups;
  const int64_t n = a.gs;
  const T* xr = x + unit * n;
  T* yr = y + unit * n;
  const int64_t step = (int64_t)kWave * EPV;
  float v[EPV];
  float s = 0.f;
  for (int64_t col = (int64_t)lane * EPV; col < n; col += step) {
    load_chunk<T, EPV>(xr, n, col, v, 0.f);
#pragma unroll
    for (int e = 0; e < EPV; ++e) s += v[e];
  }
  const float mean = wave_sum(s) / (float)n;
  float q = 0.f;
  for (int64_t col = (int64_t)lane * EPV; col < n; col += step) {
    load_chunk<T, EPV>(xr, n, col, v, 0.f);
#pragma unroll
    for (int e = 0; e < EPV; ++e)
      if (col + e < n) q += (v[e] - mean) * (v[e] - mean);
  }
  const float r = rsqrtf(wave_sum(q) / (float)n + a.eps);
  for (int64_t col = (int64_t)lane * EPV; col < n; col += step) {
    load_chunk<T, EPV>(xr, n, col, v, 0.f);
    float ex[EPV];
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      ex[e] = 0.f;
      if (col + e < n) v[e] = group_norm_pre(a, v[e] - mean, r, g * n + col + e, ex[e]);
    }
    group_norm_finish<EPV, PROG>(a, v, ex);
    store_chunk<T, EPV>(yr, n, col, v);
  }
}

// ---------------------------------------------------------------------------
// Row reductions read each element once: streaming is their natural form.
// mode 0: sum x; mode 1: sum x * v (v f32); mode 2: sum x * v (v of type T).
// A reduction's epilogue: an activation code (and its argument) or a program.
struct RowEpilogue {
  int act;
  float arg;
  hmx_program prog;
};

template <typename T, int EPV, int MODE>
__global__ __launch_bounds__(kBlock) void row_reduce(const T* x,
                                                     const void* __restrict__ vec,
                                                     T* y, int64_t m,
                                                     int64_t n, RowEpilogue epi) {
  const int64_t row = unit_index();
  if (row >= m) return;
  const int lane = threadIdx.x & (kWave - 1);
  const T* xr = x + row * n;
  const int64_t step = (int64_t)kWave * EPV;
  float v[EPV];
  float s = 0.f;
  for (int64_t col = (int64_t)lane * EPV; col < n; col += step) {
    load_chunk<T, EPV>(xr, n, col, v, 0.f);
    if constexpr (MODE == 0) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) s += v[e];
    } else if constexpr (MODE == 1) {
      float u[EPV];
      load_f32_run<EPV>((const float*)vec, n, col, u);
#pragma unroll
      for (int e = 0; e < EPV; ++e) s += v[e] * u[e];
    } else {
      float u[EPV];
      load_chunk<T, EPV>((const T*)vec, n, col, u, 0.f);
#pragma unroll
      for (int e = 0; e < EPV; ++e) s += v[e] * u[e];
    }
  }
  s = wave_sum(s);
  s = epi.act == HMX_EPI_PROGRAM ? run_program(epi.prog, s, 0.f) : apply_activation(epi.act, s, epi.arg);
  if (lane == 0) Elem<T>::store(y + row, s);
}

// Column sums in two passes, so that every CU streams rows and the result
// does not depend on scheduling. Pass 1: workgroup (b, c) sums the rows of
// chunk c for the TC * EPV columns of block b: TC threads across the columns
// (one 16-byte vector each; TC = 64 reads a contiguous 1 KiB piece of every
// row, where 128-byte pieces streamed ~20% slower) times 256 / TC threads
// down the rows, eight rows in flight per thread; the threads' sums are then
// added in thread order through LDS. The chunk's sums go to `part`
// ([chunks, n] f32), or straight to y (+ 0.0) when there is one chunk.
// Pass 2 adds the chunks in chunk order.
template <typename T, int EPV, int TC>
__global__ __launch_bounds__(256) void column_partial_kernel(const T* x, float* __restrict__ part,
                                                             int64_t m, int64_t n, int64_t rows_per_chunk,
                                                             bool final) {
  constexpr int CB = TC * EPV, TR = 256 / TC, U = 8;
  __shared__ float sums[TR][CB];
  const int tc = threadIdx.x % TC, tr = threadIdx.x / TC;
  const int64_t col = (int64_t)blockIdx.x * CB + tc * EPV;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_chunk;
  const int64_t r1 = min(m, r0 + rows_per_chunk);
  float acc[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) acc[e] = 0.f;
  if (col < n) {
    int64_t r = r0 + tr;
    for (; r + (U - 1) * TR < r1; r += U * TR) {
      float v[U][EPV];
#pragma unroll
      for (int u = 0; u < U; ++u) load_chunk<T, EPV>(x + (r + u * TR) * n, n, col, v[u], 0.f);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[e] += v[u][e];
    }
    for (; r < r1; r += TR) {
      float v[EPV];
      load_chunk<T, EPV>(x + r * n, n, col, v, 0.f);
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[e] += v[e];
    }
  }
#pragma unroll
  for (int e = 0; e < EPV; ++e) sums[tr][tc * EPV + e] = acc[e];
  __syncthreads();
  for (int k = threadIdx.x; k < CB; k += 256) {
    const int64_t c = (int64_t)blockIdx.x * CB + k;
    float t = sums[0][k];
    for (int q = 1; q < TR; ++q) t += sums[q][k];
    if (c < n) {
      if (final) part[c] = t + 0.f;
      else part[blockIdx.y * n + c] = t;
    }
  }
}

// Pass 2: each column's chunk sums in chunk order, split over kFinalSplit
// threads per column (thread t adds its run of consecutive chunks in order,
// eight loads in flight) whose sums are added in t order through LDS: a
// fixed order, so the result is the same on every run.
constexpr int kFinalCols = 32, kFinalSplit = 8;

__global__ __launch_bounds__(256) void column_final_kernel(const float* __restrict__ part,
                                                           float* __restrict__ y, int64_t chunks,
                                                           int64_t n) {
  __shared__ float red[kFinalSplit][kFinalCols];
  const int lc = threadIdx.x % kFinalCols, t = threadIdx.x / kFinalCols;
  const int64_t c = (int64_t)blockIdx.x * kFinalCols + lc;
  const int64_t per = (chunks + kFinalSplit - 1) / kFinalSplit;
  const int64_t q1 = min(chunks, (t + 1) * per);
  float s = 0.f;
  if (c < n) {
    int64_t q = t * per;
    for (; q + 8 <= q1; q += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[(q + u) * n + c];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; q < q1; ++q) s += part[q * n + c];
  }
  red[t][lc] = s;
  __syncthreads();
  if (t == 0 && c < n) {
    float v = red[0][lc];
#pragma unroll
    for (int u = 1; u < kFinalSplit; ++u) v += red[u][lc];
    y[c] = v + 0.f;
  }
}

// Elementwise ops over 16-byte vectors (EPV elements), scalar tail.
template <typename T, int EPV>
__global__ __launch_bounds__(256) void elementwise_kernel(const T* x,
                                                          T* y, int64_t numel,
                                                          int op, float arg) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * EPV;
  for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * EPV; i < numel;
       i += stride) {
    float v[EPV];
    load_chunk<T, EPV>(x, numel, i, v, 0.f);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      if (op == HMX_ELT_RELU)
        v[e] = apply_activation(HMX_EPI_RELU, v[e], 0.f);
      else if (op == HMX_ELT_LEAKY_RELU)
        v[e] = v[e] > 0.f ? v[e] : v[e] * arg;
      else
        v[e] = v[e] * arg;
    }
    store_chunk<T, EPV>(y, numel, i, v);
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.

// Layout of a cached row kernel for rows of n elements in vectors of epv:
// rows of at most 64 vectors take the smallest power-of-two lane group that
// holds them (one vector per lane; e.g. GroupNorm's 128-channel bf16 groups:
// four groups per wave); rows of up to 128 vectors one wave (two vectors per
// lane); longer rows a workgroup of tpr / 64 waves with two vectors per
// lane, doubling up to 16 waves, then more vectors per lane up to kMaxPerLane
// values. vpl == 0: the row needs the streaming kernel.
struct RowShape {
  int tpr;  // threads per row (a power of two; up to 64 * kMaxWavesPerRow)
  int vpl;
  bool whole;  // n == tpr * vpl * epv with 16-byte vectors: no guards
};

RowShape row_shape(int64_t n, int epv) {
  const int64_t vecs = ceil_div(n, epv);
  RowShape r{kWave, 0, false};
  if (vecs <= kWave) {
    // The smallest lane group holding the row: 64 / tpr rows per wave.
    r.vpl = 1;
    r.tpr = 1;
    while (r.tpr < vecs) r.tpr *= 2;
  } else if (vecs <= 2 * kWave) {
    r.vpl = 2;
  } else {
    r.tpr = 2 * kWave;
    while (r.tpr < kMaxWavesPerRow * kWave && (int64_t)r.tpr * 2 < vecs) r.tpr *= 2;
    for (int vpl = 2; vpl * epv <= kMaxPerLane; vpl *= 2)
      if ((int64_t)r.tpr * vpl >= vecs) {
        r.vpl = vpl;
        break;
      }
  }
  r.whole = r.vpl > 0 && epv > 1 && n == (int64_t)r.tpr * r.vpl * epv;
  return r;
}

// Workgroups and threads per workgroup of a cached kernel over `units` rows.
int64_t row_grid(int64_t units, const RowShape& r) {
  return r.tpr <= kWave ? ceil_div(units, kBlock / r.tpr) : units;
}
unsigned row_block(const RowShape& r) { return r.tpr <= kWave ? kBlock : r.tpr; }

// bf16 RMSNorm rows of more than 64 threads take two rows per workgroup
// unless the environment sets HMX_RMS_TWO_ROWS=0 (one, for comparison).
bool rms_two_rows() {
  static const bool on = [] {
    const char* e = getenv("HMX_RMS_TWO_ROWS");
    return !(e && e[0] == '0');
  }();
  return on;
}

template <int V>
using IntC = std::integral_constant<int, V>;

// Calls f(IntC<VPL>) for the runtime vpl (a power of two, VPL * EPV <= kMaxPerLane).
template <int EPV, typename F>
void with_vpl(int vpl, F&& f) {
  switch (vpl) {
    case 1: f(IntC<1>{}); break;
    case 2: f(IntC<2>{}); break;
    case 4: if constexpr (4 * EPV <= kMaxPerLane) f(IntC<4>{}); break;
    case 8: if constexpr (8 * EPV <= kMaxPerLane) f(IntC<8>{}); break;
    case 16: if constexpr (16 * EPV <= kMaxPerLane) f(IntC<16>{}); break;
  }
}

// Calls f(IntC<VPL>, bool_constant<WHOLE>) for a cached row shape.
template <int EPV, typename F>
void with_shape(const RowShape& r, F&& f) {
  with_vpl<EPV>(r.vpl, [&](auto vpl_c) {
    if constexpr (EPV > 1) {
      if (r.whole) {
        f(vpl_c, std::true_type{});
        return;
      }
    }
    f(vpl_c, std::false_type{});
  });
}

// Calls f(T*, IntC<EPV>) for the dtype and whether 16-byte vectors apply.
template <typename F>
void with_type(int dtype, bool vec, F&& f) {
  if (dtype == HMX_DTYPE_BF16) {
    if (vec) f((uint16_t*)nullptr, IntC<8>{});
    else f((uint16_t*)nullptr, IntC<1>{});
  } else {
    if (vec) f((float*)nullptr, IntC<4>{});
    else f((float*)nullptr, IntC<1>{});
  }
}

// Whether rows of `n` elements starting at `p` (and `q`) keep 16-byte alignment.
bool rows_vectorizable(const void* p, const void* q, int64_t n, int dtype) {
  const int64_t epv = 16 / dtype_bytes(dtype);
  return aligned16(p) && aligned16(q) && n % epv == 0;
}

dim3 unit_grid(int64_t units) { return dim3((unsigned)ceil_div(units, kRowsPerBlock)); }

// How many workgroups of `block` threads of `kernel` one CU holds at once,
// read from the runtime once per kernel and block size (1 if it cannot say).
// A kernel whose workgroups walk many rows launches no more than fit, so
// that none waits for another to finish.
template <auto Kernel>
int resident_blocks(int block) {
  static std::atomic<int> known[5];  // block = 64 << i
  int i = 0;
  while (i < 4 && (kWave << i) < block) ++i;
  int b = known[i].load(std::memory_order_relaxed);
  if (b > 0) return b;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, Kernel, block, 0) != hipSuccess || b < 1) {
    (void)hipGetLastError();
    b = 1;
  }
  known[i].store(b, std::memory_order_relaxed);
  return b;
}

// The largest workgroup count of a one-dimensional launch.
constexpr int64_t kMaxGrid = 0x7fffffff;

}  // namespace
}  // namespace hmx

using namespace hmx;

extern "C" {

int hmx_softmax_rows(int dtype, const void* x, void* y, int64_t m, int64_t n,
                     void* stream) {
  HMX_REQUIRE(valid_dtype(dtype), "softmax: unknown dtype %d", dtype);
  HMX_REQUIRE(m >= 0 && n >= 1, "softmax: invalid shape [%lld, %lld]", (long long)m,
              (long long)n);
  HMX_REQUIRE(x && y, "softmax: null operand");
  HMX_REQUIRE(m <= kMaxGrid, "softmax: too many rows");
  if (m == 0) return HMX_OK;
  auto s = (hipStream_t)stream;
  with_type(dtype, rows_vectorizable(x, y, n, dtype), [&](auto tp, auto epv_c) {
    using T = std::remove_pointer_t<decltype(tp)>;
    constexpr int EPV = decltype(epv_c)::value;
    const RowShape r = row_shape(n, EPV);
    if (r.vpl == 0) {
      launch(softmax_stream<T, EPV>, unit_grid(m), kBlock, s, (const T*)x, (T*)y, m, n);
      return;
    }
    with_shape<EPV>(r, [&](auto vpl_c, auto whole_c) {
      launch(softmax_cached<T, EPV, decltype(vpl_c)::value, decltype(whole_c)::value>,
             dim3((unsigned)row_grid(m, r)), row_block(r), s, (const T*)x, (T*)y, m, n, r.tpr);
    });
  });
  return check_launch("softmax");
}

int hmx_rmsnorm_rows(int dtype, const void* x, const void* w, int w_dtype, void* y,
                     int64_t m, int64_t n, float eps, void* stream) {
  HMX_REQUIRE(valid_dtype(dtype) && (w == nullptr || valid_dtype(w_dtype)),
              "rms_norm: unknown dtype");
  HMX_REQUIRE(m >= 0 && n >= 1, "rms_norm: invalid shape [%lld, %lld]", (long long)m,
              (long long)n);
  HMX_REQUIRE(x && y, "rms_norm: null operand");
  HMX_REQUIRE(m <= kMaxGrid, "rms_norm: too many rows");
  if (m == 0) return HMX_OK;
  auto s = (hipStream_t)stream;
  const bool w_vec = aligned16(w);
  with_type(dtype, rows_vectorizable(x, y, n, dtype), [&](auto tp, auto epv_c) {
    using T = std::remove_pointer_t<decltype(tp)>;
    constexpr int EPV = decltype(epv_c)::value;
    auto with_weight = [&](auto wp) {
      using W = std::remove_pointer_t<decltype(wp)>;
      const RowShape r = row_shape(n, EPV);
      if (r.vpl == 0) {
        launch(rmsnorm_stream<T, W, EPV>, unit_grid(m), kBlock, s, (const T*)x, (const W*)w, w_vec,
               (T*)y, m, n, eps);
        return;
      }
      with_shape<EPV>(r, [&](auto vpl_c, auto whole_c) {
        constexpr int VPLc = decltype(vpl_c)::value;
        constexpr bool WH = decltype(whole_c)::value;
        // Two rows per workgroup for bf16 rows (config 2: 76.3 -> 75.6 us);
        // f32 rows measured slower that way (169 -> 177 us).
        if (r.tpr > kWave && sizeof(T) == 2 && rms_two_rows())
          launch(rmsnorm_cached2<T, W, EPV, VPLc, WH>, dim3((unsigned)ceil_div(m, 2)), row_block(r), s,
                 (const T*)x, (const W*)w, w_vec, (T*)y, m, n, eps, r.tpr);
        else
          launch(rmsnorm_cached<T, W, EPV, VPLc, WH>, dim3((unsigned)row_grid(m, r)), row_block(r), s,
                 (const T*)x, (const W*)w, w_vec, (T*)y, m, n, eps, r.tpr);
      });
    };
    if (w != nullptr && w_dtype == HMX_DTYPE_BF16)
      with_weight((uint16_t*)nullptr);
    else
      with_weight((float*)nullptr);
  });
  return check_launch("rms_norm");
}

int hmx_group_norm_rows(int dtype, const void* x, const void* w, const void* b,
                        const void* extra, int vec_dtype, void* y, int64_t m,
                        int64_t groups, int64_t group_size, float eps, int extra_op,
                        int activation, float activation_arg, const hmx_program* program,
                        void* stream) {
  HMX_REQUIRE(valid_dtype(dtype) && valid_dtype(vec_dtype), "group_norm: unknown dtype");
  HMX_REQUIRE(m >= 0 && groups >= 1 && group_size >= 1, "group_norm: invalid shape");
  HMX_REQUIRE(x && y, "group_norm: null operand");
  HMX_REQUIRE(extra_op >= HMX_EXTRA_NONE && extra_op <= HMX_EXTRA_MUL,
              "group_norm: unknown extra op %d", extra_op);
  HMX_REQUIRE(extra_op == HMX_EXTRA_NONE || extra != nullptr,
              "group_norm: extra op without an extra operand");
  hmx_program prog;
  const int pst = check_epilogue("group_norm", activation, program, &prog);
  if (pst != HMX_OK) return pst;
  HMX_REQUIRE(activation != HMX_EPI_PROGRAM || extra_op == HMX_EXTRA_NONE,
              "group_norm: an epilogue program reads the extra operand itself (extra op must be none)");
  const int64_t units = m * groups;
  HMX_REQUIRE(units <= kMaxGrid, "group_norm: too many rows");
  if (units == 0) return HMX_OK;
  GroupNormArgs a{};
  a.w = w;
  a.b = b;
  a.extra = extra;
  a.vec_dtype = vec_dtype;
  a.units = units;
  a.groups = groups;
  a.gs = group_size;
  a.eps = eps;
  a.extra_op = extra_op;
  a.act = activation;
  a.act_arg = activation_arg;
  a.prog = prog;
  a.vec_ok = aligned16(w) && aligned16(b) && aligned16(extra);
  auto s = (hipStream_t)stream;
  with_type(dtype, rows_vectorizable(x, y, group_size, dtype), [&](auto tp, auto epv_c) {
    using T = std::remove_pointer_t<decltype(tp)>;
    constexpr int EPV = decltype(epv_c)::value;
    const RowShape r = row_shape(group_size, EPV);
    if constexpr (EPV > 1) {
      // Whole rows in registers when the row fits and each group is one run
      // of aligned lanes (or the whole row): w, b and extra stay resident.
      const int64_t row_n = groups * group_size;
      const RowShape rr = row_shape(row_n, EPV);
      const int64_t gv = group_size / EPV;
      const bool one = groups == 1;
      // A program's interpreter needs more than the 128 VGPRs of a
      // 1024-thread workgroup: its kernels are built for rows of at most
      // kProgBlock threads.
      const bool fits = activation != HMX_EPI_PROGRAM || row_block(rr) <= (unsigned)kProgBlock;
      const bool whole_rows = a.vec_ok && rr.vpl > 0 && rr.whole && (one || ((gv & (gv - 1)) == 0 && gv <= rr.tpr));
      // A program compiled into the kernel at run time: no interpreter, so
      // every whole-row shape (workgroups of up to 16 waves) takes it.
      if (whole_rows && activation == HMX_EPI_PROGRAM &&
          launch_group_norm_jit(std::is_same_v<T, uint16_t>, x, y, a, m, rr.tpr, (int)gv, EPV, rr.vpl, one,
                                extra != nullptr, row_block(rr), rr.tpr <= kWave ? (int)(kBlock / rr.tpr) : 1,
                                current_device_shape().cus, s) == HMX_OK)
        return;
      if (whole_rows && fits) {
        const int rpb = rr.tpr <= kWave ? (int)(kBlock / rr.tpr) : 1;
        const unsigned block = row_block(rr);
        with_vpl<EPV>(rr.vpl, [&](auto vpl_c) {
          constexpr int VPL = decltype(vpl_c)::value;
          auto go = [&](auto one_c, auto extra_c, auto prog_c) {
            constexpr auto kernel = &group_norm_rows<T, EPV, VPL, decltype(one_c)::value, decltype(extra_c)::value,
                                                     decltype(prog_c)::value>;
            // As many workgroups as the GPU holds at once, each walking rows
            // blockIdx, blockIdx + grid, ...
            const int64_t resident = (int64_t)resident_blocks<kernel>((int)block) * current_device_shape().cus;
            launch(kernel, dim3((unsigned)std::min(ceil_div(m, rpb), resident)), block, s, (const T*)x, (T*)y, a,
                   m, rr.tpr, (int)gv);
          };
          // With a program, EXTRA: an extra operand is given (the program
          // reads it); else: an extra op applies.
          const bool program = activation == HMX_EPI_PROGRAM;
          const bool has_extra = program ? extra != nullptr : extra_op != HMX_EXTRA_NONE;
          auto go2 = [&](auto one_c) {
            if (program) {
              if (has_extra) go(one_c, std::true_type{}, std::true_type{});
              else go(one_c, std::false_type{}, std::true_type{});
            } else {
              if (has_extra) go(one_c, std::true_type{}, std::false_type{});
              else go(one_c, std::false_type{}, std::false_type{});
            }
          };
          if (one) go2(std::true_type{});
          else go2(std::false_type{});
        });
        return;
      }
    }
    if (activation == HMX_EPI_PROGRAM) {
      // Programs on rows the whole-row kernel does not take run in the
      // streaming kernel: the cached kernels stay free of the interpreter's
      // registers.
      launch(group_norm_stream<T, EPV, true>, unit_grid(units), kBlock, s, (const T*)x, (T*)y, a);
      return;
    }
    if (r.vpl == 0) {
      launch(group_norm_stream<T, EPV, false>, unit_grid(units), kBlock, s, (const T*)x, (T*)y, a);
      return;
    }
    with_shape<EPV>(r, [&](auto vpl_c, auto whole_c) {
      launch(group_norm_cached<T, EPV, decltype(vpl_c)::value, decltype(whole_c)::value>,
             dim3((unsigned)row_grid(units, r)), row_block(r), s, (const T*)x, (T*)y, a, r.tpr);
    });
  });
  return check_launch("group_norm");
}

static int row_reduce_launch(const char* name, int mode, int dtype, const void* x,
                             const void* vec, void* y, int64_t m, int64_t n, int act,
                             float act_arg, const hmx_program* program, void* stream) {
  HMX_REQUIRE(valid_dtype(dtype), "%s: unknown dtype %d", name, dtype);
  HMX_REQUIRE(m >= 0 && n >= 0, "%s: invalid shape", name);
  // Rows of no columns read nothing: x and vec may then be null (an empty
  // tensor's data pointer).
  HMX_REQUIRE((x || n == 0) && y && (mode == 0 || vec || n == 0), "%s: null operand", name);
  RowEpilogue epi{act, act_arg, {}};
  const int pst = check_epilogue(name, act, program, &epi.prog);
  if (pst != HMX_OK) return pst;
  HMX_REQUIRE(m <= ((int64_t)1 << 31) * kRowsPerBlock, "%s: too many rows", name);
  if (m == 0) return HMX_OK;
  auto s = (hipStream_t)stream;
  bool vec_ok = rows_vectorizable(x, x, n, dtype);
  if (mode != 0) vec_ok = vec_ok && aligned16(vec);
  with_type(dtype, vec_ok, [&](auto tp, auto epv_c) {
    using T = std::remove_pointer_t<decltype(tp)>;
    constexpr int EPV = decltype(epv_c)::value;
    if (mode == 0)
      launch(row_reduce<T, EPV, 0>, unit_grid(m), kBlock, s, (const T*)x, vec, (T*)y, m, n, epi);
    else if (mode == 1)
      launch(row_reduce<T, EPV, 1>, unit_grid(m), kBlock, s, (const T*)x, vec, (T*)y, m, n, epi);
    else
      launch(row_reduce<T, EPV, 2>, unit_grid(m), kBlock, s, (const T*)x, vec, (T*)y, m, n, epi);
  });
  return check_launch(name);
}

int hmx_row_sum(int dtype, const void* x, void* y, int64_t m, int64_t n, int activation,
                float activation_arg, const hmx_program* program, void* stream) {
  return row_reduce_launch("row_sum", 0, dtype, x, nullptr, y, m, n, activation,
                           activation_arg, program, stream);
}

int hmx_row_dot(int dtype, const void* x, const float* v, void* y, int64_t m, int64_t n,
                int activation, float activation_arg, const hmx_program* program, void* stream) {
  return row_reduce_launch("row_dot", 1, dtype, x, v, y, m, n, activation, activation_arg,
                           program, stream);
}

int hmx_matvec(int dtype, const void* a, const void* x, void* y, int64_t m, int64_t k,
               void* stream) {
  return row_reduce_launch("matvec", 2, dtype, a, x, y, m, k, HMX_EPI_IDENTITY, 0.f, nullptr, stream);
}

// Row chunks of a column sum: about 2048 workgroups, at least 256 rows each.
// Row chunks of pass 1: about 1024 workgroups over the column blocks of
// 512 columns, at least 256 rows per chunk.
static void column_chunks(int64_t m, int64_t n, int64_t& chunks, int64_t& rows_per_chunk) {
  const int64_t blocks = std::max<int64_t>(1, ceil_div(n, 512));
  chunks = std::max<int64_t>(1, std::min(ceil_div(1024, blocks), ceil_div(m, 256)));
  rows_per_chunk = ceil_div(m, chunks);
  chunks = rows_per_chunk > 0 ? ceil_div(m, rows_per_chunk) : 1;
}

int hmx_column_sum_plan(int64_t m, int64_t n, int64_t* workspace_bytes) {
  HMX_REQUIRE(m >= 0 && n >= 0 && workspace_bytes, "column_sum_plan: invalid arguments");
  int64_t chunks, rows;
  column_chunks(m, n, chunks, rows);
  *workspace_bytes = chunks > 1 ? chunks * n * (int64_t)sizeof(float) : 0;
  return HMX_OK;
}

int hmx_column_sum(int dtype, const void* x, float* y, int64_t m, int64_t n, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  HMX_REQUIRE(valid_dtype(dtype), "column_sum: unknown dtype %d", dtype);
  HMX_REQUIRE(m >= 0 && n >= 0, "column_sum: invalid shape");
  HMX_REQUIRE((x || m == 0) && y, "column_sum: null operand");  // no rows: x is not read
  if (n == 0) return HMX_OK;
  int64_t chunks, rows;
  column_chunks(m, n, chunks, rows);
  HMX_REQUIRE(chunks <= 65535 && ceil_div(n, 8) <= kMaxGrid, "column_sum: too many columns");
  const int64_t need = chunks > 1 ? chunks * n * (int64_t)sizeof(float) : 0;
  HMX_REQUIRE(need == 0 || (workspace && workspace_bytes >= need),
              "column_sum: workspace of %lld bytes needed (hmx_column_sum_plan), %lld given",
              (long long)need, (long long)workspace_bytes);
  auto s = (hipStream_t)stream;
  float* part = chunks > 1 ? (float*)workspace : y;
  with_type(dtype, rows_vectorizable(x, x, n, dtype), [&](auto tp, auto epv_c) {
    using T = std::remove_pointer_t<decltype(tp)>;
    constexpr int EPV = decltype(epv_c)::value;
    // The fewest threads across (8 to 64) whose vectors span the row.
    const int64_t vecs = ceil_div(n, EPV);
    auto go = [&](auto tc_c) {
      constexpr int TC = decltype(tc_c)::value;
      const dim3 grid((unsigned)ceil_div(n, TC * EPV), (unsigned)chunks);
      launch(column_partial_kernel<T, EPV, TC>, grid, 256, s, (const T*)x, part, m, n, rows, chunks == 1);
    };
    if (vecs <= 8) go(IntC<8>{});
    else if (vecs <= 16) go(IntC<16>{});
    else if (vecs <= 32) go(IntC<32>{});
    else go(IntC<64>{});
  });
  if (chunks > 1)
    launch(column_final_kernel, dim3((unsigned)ceil_div(n, kFinalCols)), 256, s, (const float*)part, y, chunks,
           n);
  return check_launch("column_sum");
}

int hmx_elementwise(int op, int dtype, const void* x, void* y, int64_t numel, float arg,
                    void* stream) {
  HMX_REQUIRE(valid_dtype(dtype), "elementwise: unknown dtype %d", dtype);
  HMX_REQUIRE(op >= HMX_ELT_RELU && op <= HMX_ELT_SCALE, "elementwise: unknown op %d", op);
  HMX_REQUIRE(numel >= 0, "elementwise: negative size");
  HMX_REQUIRE(x && y, "elementwise: null operand");
  if (numel == 0) return HMX_OK;
  auto s = (hipStream_t)stream;
  const bool vec = aligned16(x) && aligned16(y);
  with_type(dtype, vec, [&](auto tp, auto epv_c) {
    using T = std::remove_pointer_t<decltype(tp)>;
    constexpr int EPV = decltype(epv_c)::value;
    const int64_t blocks = std::min<int64_t>(ceil_div(numel, 256 * EPV), 8192);
    launch(elementwise_kernel<T, EPV>, dim3((unsigned)blocks), 256, s, (const T*)x, (T*)y, numel,
           op, arg);
  });
  return check_launch("elementwise");
}

}  // extern "C"
