// Row-kernel pieces shared by the library's row kernels (hmx_rows.hip) and
// the whole-row GroupNorm kernels hmx_jit.cpp compiles at run time with an
// epilogue program compiled in: row access, reductions, GroupNormArgs and
// the whole-row GroupNorm body.
#pragma once

#include <type_traits>

#include "hmx_device.hpp"

namespace hmx {

// The run-time compiled epilogue: f(value, extra). Only the sources that
// hmx_jit.cpp compiles define it.
__device__ float hmx_jit_epilogue(float x, float extra);

// ---------------------------------------------------------------------------
// GroupNorm over units of `gs` elements (row r, group g at r * G * gs + g * gs):
// mean, centered variance, ((x - mean) * rsqrt(var + eps)) * w + b, then the
// extra operand and activation; normalization.py:113-122.
struct GroupNormArgs {
  const void* w;
  const void* b;
  const void* extra;
  int vec_dtype;
  int64_t units;
  int64_t groups;
  int64_t gs;
  float eps;
  int extra_op;
  int act;
  float act_arg;
  hmx_program prog;  // act == HMX_EPI_PROGRAM: the whole epilogue, y = prog(value, extra)
  // w, b and extra are 16-byte aligned: with vectorizable rows (gs a
  // multiple of EPV), each row vector's EPV channels load as one piece.
  bool vec_ok;
};

#ifndef __HIPCC_RTC__
// hmx_jit.cpp: the whole-row GroupNorm kernel (T = bf16 bits or f32, EPV,
// VPL, ONE, EXTRA as group_norm_rows_body) with a's epilogue program compiled
// in, `block` threads per workgroup of `rows_per_block` rows, as many
// workgroups as the device's `cus` compute units hold at once. HMX_OK, or
// HMX_ERR_UNSUPPORTED when run-time compilation is off (HMX_JIT=0) or failed:
// the caller then launches the interpreter.
int launch_group_norm_jit(bool bf16, const void* x, void* y, const GroupNormArgs& a, int64_t rows, int tpr,
                          int gv, int epv, int vpl, bool one, bool extra, unsigned block, int rows_per_block,
                          int cus, hipStream_t stream);
#endif

namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kBlock = kRowsPerBlock * kWave;
// f32 values a lane keeps of a cached row: 16 VGPRs, so that every cached
// kernel fits a 1024-thread workgroup (128 VGPRs per lane at most) without
// spilling. Rows of up to 16 waves x 64 lanes x 16 = 16384 values are cached.
constexpr int kMaxPerLane = 16;
// Waves of a workgroup that share one row.
constexpr int kMaxWavesPerRow = 16;
constexpr int kMaxBlock = kMaxWavesPerRow * kWave;
// Workgroups of kernels that run an epilogue program: two waves per SIMD at
// most, 256 VGPRs each.
constexpr int kProgBlock = 8 * kWave;

// ---------------------------------------------------------------------------
// Row access. `tpr` threads share a row; thread `li` of them holds, as its
// j-th vector, columns [(j * tpr + li) * EPV, ... + EPV): for each j the
// threads read one contiguous tpr * EPV run, so every load instruction is
// fully coalesced.
// WHOLE: n == tpr * VPL * EPV, every vector is in the row (no guards).
template <typename T, int EPV, int VPL, bool WHOLE = false>
__device__ __forceinline__ void load_row(const T* __restrict__ p, int64_t n, int li, int tpr,
                                         float (&v)[VPL * EPV], float fill) {
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t col = ((int64_t)j * tpr + li) * EPV;
    if constexpr (EPV > 1) {
      if (WHOLE || col + EPV <= n) {
        uint4 raw;
        if constexpr (std::is_same_v<T, float>) {
          // f32 rows: non-temporal loads measure 2-3% more bandwidth on
          // [32768, 4096] softmax/RMSNorm; for bf16 rows they cost 8-12%.
          const u32x4_t nt = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p + col));
          raw = make_uint4(nt[0], nt[1], nt[2], nt[3]);
        } else {
          raw = *reinterpret_cast<const uint4*>(p + col);
        }
        Elem<T>::unpack(raw, &v[j * EPV]);
      } else {
#pragma unroll
        for (int e = 0; e < EPV; ++e)
          v[j * EPV + e] = (col + e < n) ? Elem<T>::load(p + col + e) : fill;
      }
    } else {
      v[j] = col < n ? Elem<T>::load(p + col) : fill;
    }
  }
}

template <typename T, int EPV, int VPL, bool WHOLE = false>
__device__ __forceinline__ void store_row(T* __restrict__ p, int64_t n, int li, int tpr,
                                          const float (&v)[VPL * EPV]) {
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t col = ((int64_t)j * tpr + li) * EPV;
    if constexpr (EPV > 1) {
      if (WHOLE || col + EPV <= n) {
        store16_stream(p + col, Elem<T>::pack(&v[j * EPV]));
      } else {
#pragma unroll
        for (int e = 0; e < EPV; ++e)
          if (col + e < n) Elem<T>::store(p + col + e, v[j * EPV + e]);
      }
    } else {
      if (col < n) Elem<T>::store(p + col, v[j]);
    }
  }
}

// Column of element e of a thread's j-th vector.
template <int EPV>
__device__ __forceinline__ int64_t col_of(int j, int li, int tpr, int e) {
  return ((int64_t)j * tpr + li) * EPV + e;
}

// Where a thread of a cached-row kernel sits: `tpr` threads per row, a power
// of two. tpr <= 64: 64 / tpr rows per wave (aligned lane groups) and
// blockDim.x / tpr rows per workgroup; tpr > 64: tpr / 64 waves per row, one
// row per workgroup.
struct RowPos {
  int64_t row;
  int li;   // index among the row's threads
  int tpr;  // threads per row
};

__device__ __forceinline__ RowPos row_pos(int tpr) {
  return RowPos{(int64_t)blockIdx.x * (blockDim.x / tpr) + threadIdx.x / tpr, (int)(threadIdx.x % tpr), tpr};
}

// Sum / max over all threads of a row: xor butterflies within the row's lane
// group (offsets below min(tpr, 64)), then (tpr > 64) the waves' partials
// through LDS, combined in wave order by every thread, so all threads hold the
// same value. Each call site passes its own `slot` array (kMaxWavesPerRow
// floats): no slot is written twice.
__device__ __forceinline__ float row_sum_all(float v, float* slot, int tpr) {
  for (int off = (tpr < kWave ? tpr : kWave) >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  if (tpr > kWave) {
    if ((threadIdx.x & (kWave - 1)) == 0) slot[threadIdx.x >> 6] = v;
    __syncthreads();
    v = slot[0];
    for (int q = 1; q < tpr / kWave; ++q) v += slot[q];
  }
  return v;
}

__device__ __forceinline__ float row_max_all(float v, float* slot, int tpr) {
  for (int off = (tpr < kWave ? tpr : kWave) >> 1; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  if (tpr > kWave) {
    if ((threadIdx.x & (kWave - 1)) == 0) slot[threadIdx.x >> 6] = v;
    __syncthreads();
    v = slot[0];
    for (int q = 1; q < tpr / kWave; ++q) v = fmaxf(v, slot[q]);
  }
  return v;
}

// Streaming access for rows longer than the register cache: chunk c of a row
// is the c-th run of 64 * EPV columns.
template <typename T, int EPV>
__device__ __forceinline__ void load_chunk(const T* __restrict__ p, int64_t n, int64_t col,
                                           float (&v)[EPV], float fill) {
  if constexpr (EPV > 1) {
    if (col + EPV <= n) {
      Elem<T>::unpack(*reinterpret_cast<const uint4*>(p + col), v);
      return;
    }
  }
#pragma unroll
  for (int e = 0; e < EPV; ++e) v[e] = (col + e < n) ? Elem<T>::load(p + col + e) : fill;
}

template <typename T, int EPV>
__device__ __forceinline__ void store_chunk(T* __restrict__ p, int64_t n, int64_t col,
                                            const float (&v)[EPV]) {
  if constexpr (EPV > 1) {
    if (col + EPV <= n) {
      store16_stream(p + col, Elem<T>::pack(v));
      return;
    }
  }
#pragma unroll
  for (int e = 0; e < EPV; ++e)
    if (col + e < n) Elem<T>::store(p + col + e, v[e]);
}

// EPV consecutive f32 values (zero past n), as 16-byte loads where they fit.
template <int EPV>
__device__ __forceinline__ void load_f32_run(const float* __restrict__ p, int64_t n,
                                             int64_t col, float (&u)[EPV]) {
  if constexpr (EPV % 4 == 0) {
    if (col + EPV <= n) {
#pragma unroll
      for (int q = 0; q < EPV / 4; ++q)
        Elem<float>::unpack(*reinterpret_cast<const uint4*>(p + col + 4 * q), &u[4 * q]);
      return;
    }
  }
#pragma unroll
  for (int e = 0; e < EPV; ++e) u[e] = (col + e < n) ? p[col + e] : 0.f;
}

// EPV consecutive values of a per-column vector of storage type W (f32 or
// bf16 bits) as f32, with 16-byte loads when `vec` (16-byte aligned base) and
// the run is whole; zero past n.
template <typename W, int EPV>
__device__ __forceinline__ void load_vec_run(const W* __restrict__ p, int64_t n, int64_t col,
                                             bool vec, float (&u)[EPV]) {
  constexpr int BYTES = EPV * (int)sizeof(W);
  constexpr int PER16 = 16 / (int)sizeof(W);
  if constexpr (BYTES % 16 == 0) {
    if (vec && col + EPV <= n) {
      const uint4* q = reinterpret_cast<const uint4*>(p + col);
#pragma unroll
      for (int i = 0; i < BYTES / 16; ++i) Elem<W>::unpack(q[i], &u[i * PER16]);
      return;
    }
  }
#pragma unroll
  for (int e = 0; e < EPV; ++e) u[e] = (col + e < n) ? Elem<W>::load(p + col + e) : 0.f;
}

__device__ __forceinline__ int64_t unit_index() {
  return (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
}

// `fill` for a null vector, else EPV consecutive values from index i (a
// multiple of EPV) of a 16-byte aligned f32 or bf16 vector, with 16-byte loads
// where the run fills them.
template <int EPV>
__device__ __forceinline__ void load_vec_any(const void* p, int dtype, int64_t i, float (&out)[EPV],
                                             float fill) {
  if (!p) {
#pragma unroll
    for (int e = 0; e < EPV; ++e) out[e] = fill;
  } else if (dtype == HMX_DTYPE_F32) {
    load_vec_run<float, EPV>((const float*)p, i + EPV, i, true, out);
  } else {
    load_vec_run<uint16_t, EPV>((const uint16_t*)p, i + EPV, i, true, out);
  }
}

// The activation on N pre-activation values in place: a named code, or with
// PROG (the kernel instantiated for epilogue programs) the program.
template <int N, bool PROG>
__device__ __forceinline__ void group_norm_finish(const GroupNormArgs& a, float (&v)[N],
                                                  const float (&extra)[N]) {
  if constexpr (PROG) {
    if (a.act == HMX_EPI_PROGRAM) {
      run_program_n<N>(a.prog, v, extra);
      return;
    }
  }
  if (a.act != HMX_EPI_IDENTITY) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = apply_activation(a.act, v[i], a.act_arg);
  }
}

// Sums of VPL per-lane values, value j over the gv lanes that hold vector j
// of one group (gv a power of two dividing the row's thread count, lanes
// aligned to it). gv > 64: the waves' partials meet in `slot` (VPL x
// kMaxWavesPerRow floats, one array per call site) and each thread adds its
// group's waves in wave order.
template <int VPL>
__device__ __forceinline__ void group_sums(float (&s)[VPL], int gv, float* slot) {
  for (int off = (gv < kWave ? gv : kWave) >> 1; off > 0; off >>= 1) {
#pragma unroll
    for (int j = 0; j < VPL; ++j) s[j] += __shfl_xor(s[j], off, kWave);
  }
  if (gv > kWave) {
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & (kWave - 1)) == 0) {
#pragma unroll
      for (int j = 0; j < VPL; ++j) slot[j * kMaxWavesPerRow + wave] = s[j];
    }
    __syncthreads();
    const int wpg = gv / kWave;
    const int w0 = wave - wave % wpg;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float t = slot[j * kMaxWavesPerRow + w0];
      for (int q = 1; q < wpg; ++q) t += slot[j * kMaxWavesPerRow + w0 + q];
      s[j] = t;
    }
  }
}

// Raw 16-byte vectors of one row, as load_row reads them (whole rows only).
template <typename T, int EPV, int VPL>
__device__ __forceinline__ void load_row_raw(const T* __restrict__ p, int li, int tpr, uint4 (&raw)[VPL]) {
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const T* q = p + ((int64_t)j * tpr + li) * EPV;
    if constexpr (std::is_same_v<T, float>) {
      const u32x4_t nt = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(q));
      raw[j] = make_uint4(nt[0], nt[1], nt[2], nt[3]);
    } else {
      raw[j] = *reinterpret_cast<const uint4*>(q);
    }
  }
}

// GroupNorm / LayerNorm over whole rows of G groups, each workgroup walking
// many rows with w, b (and the extra operand's per-channel vector) of its
// lanes' columns held in registers: they are read once per workgroup instead
// of once per row. Re-read per row, f32 w and b move 4x a bf16 row's bytes
// through L2, which then bounds the kernel rather than HBM. The next row's x
// is loaded before the current row is reduced. The row (n = G * gs channels)
// is whole: n == tpr * VPL * EPV; a group is gv = gs / EPV vectors, either
// the whole row (ONE) or a power of two dividing tpr, so vector j of a lane
// belongs to the group of the gv aligned lanes around it. Statistics are
// f32: mean, then the centered variance, per group. EPI: EPI_NAMED (a named
// activation, or none), EPI_PROGRAM (the interpreter runs the program on
// (normalized value, extra)) or EPI_JIT (hmx_jit_epilogue, compiled in at
// run time), EXTRA then meaning that an extra operand is given (else register
// 1 reads 0).
enum : int { EPI_NAMED = 0, EPI_PROGRAM = 1, EPI_JIT = 2 };

template <typename T, int EPV, int VPL, bool ONE, bool EXTRA, int EPI>
__device__ __forceinline__ void group_norm_rows_body(const T* x, T* y, const GroupNormArgs& a, int64_t rows,
                                                     int tpr, int gv) {
  constexpr bool PROG = EPI != EPI_NAMED;
  __shared__ float red_mean[VPL * kMaxWavesPerRow], red_var[VPL * kMaxWavesPerRow];
  const int rpb = tpr <= kWave ? (int)blockDim.x / tpr : 1;
  const int li = (int)threadIdx.x % tpr;
  int64_t row = (int64_t)blockIdx.x * rpb + threadIdx.x / tpr;
  const int64_t step = (int64_t)gridDim.x * rpb;
  // Threads of one row share `row` (tpr > 64: the whole workgroup), so an
  // early return never skips a barrier another thread of the row waits at.
  if (row >= rows) return;
  const int64_t n = a.gs * a.groups;
  float wv[VPL * EPV], bv[VPL * EPV], ev[EXTRA ? VPL * EPV : 1];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t col0 = col_of<EPV>(j, li, tpr, 0);
    float t[EPV];
    load_vec_any<EPV>(a.w, a.vec_dtype, col0, t, 1.f);
#pragma unroll
    for (int e = 0; e < EPV; ++e) wv[j * EPV + e] = t[e];
    load_vec_any<EPV>(a.b, a.vec_dtype, col0, t, 0.f);
#pragma unroll
    for (int e = 0; e < EPV; ++e) bv[j * EPV + e] = t[e];
    if constexpr (EXTRA) {
      load_vec_any<EPV>(a.extra, a.vec_dtype, col0, t, 0.f);
#pragma unroll
      for (int e = 0; e < EPV; ++e) ev[j * EPV + e] = t[e];
    }
  }
  const float inv_n = 1.f / (float)(ONE ? n : a.gs);
  uint4 cur[VPL];
  load_row_raw<T, EPV, VPL>(x + row * n, li, tpr, cur);
  for (;;) {
    const int64_t next = row + step;
    uint4 nxt[VPL];
    if (next < rows) load_row_raw<T, EPV, VPL>(x + next * n, li, tpr, nxt);
    float v[VPL * EPV];
#pragma unroll
    for (int j = 0; j < VPL; ++j) Elem<T>::unpack(cur[j], &v[j * EPV]);
    float mean[VPL], r[VPL];
    if constexpr (ONE) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < VPL * EPV; ++i) s += v[i];
      const float m0 = row_sum_all(s, red_mean, tpr) / (float)n;
      float q = 0.f;
#pragma unroll
      for (int i = 0; i < VPL * EPV; ++i) q += (v[i] - m0) * (v[i] - m0);
      const float r0 = rsqrtf(row_sum_all(q, red_var, tpr) / (float)n + a.eps);
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        mean[j] = m0;
        r[j] = r0;
      }
    } else {
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < EPV; ++e) s += v[j * EPV + e];
        mean[j] = s;
      }
      group_sums<VPL>(mean, gv, red_mean);
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        mean[j] *= inv_n;
        float q = 0.f;
#pragma unroll
        for (int e = 0; e < EPV; ++e) q += (v[j * EPV + e] - mean[j]) * (v[j * EPV + e] - mean[j]);
        r[j] = q;
      }
      group_sums<VPL>(r, gv, red_var);
#pragma unroll
      for (int j = 0; j < VPL; ++j) r[j] = rsqrtf(r[j] * inv_n + a.eps);
    }
    float ex[VPL * EPV];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const int i = j * EPV + e;
        float yv = (v[i] - mean[j]) * r[j] * wv[i];
        yv += bv[i];
        if constexpr (EXTRA && !PROG) {
          if (a.extra_op == HMX_EXTRA_ADD) yv += ev[i];
          if (a.extra_op == HMX_EXTRA_MUL) yv *= ev[i];
        }
        v[i] = yv;
        if constexpr (EXTRA && PROG) ex[i] = ev[i];
        else ex[i] = 0.f;
      }
    }
    if constexpr (EPI == EPI_JIT) {
#pragma unroll
      for (int i = 0; i < VPL * EPV; ++i) v[i] = hmx_jit_epilogue(v[i], ex[i]);
    } else if constexpr (PROG) {
      // The program on 8 of the lane's values at a time (its dispatch,
      // not the arithmetic, is what an instruction costs; 16 at a time
      // spilled): f32 [32768, 4096] with a 4-instruction program 543 ->
      // 429 us against one row vector (4 values) at a time.
      constexpr int P = VPL * EPV < 8 ? VPL * EPV : 8;
#pragma unroll
      for (int j = 0; j < VPL * EPV; j += P) {
        float (&vj)[P] = *reinterpret_cast<float (*)[P]>(&v[j]);
        const float (&ej)[P] = *reinterpret_cast<const float (*)[P]>(&ex[j]);
        run_program_n<P>(a.prog, vj, ej);
      }
    } else {
      group_norm_finish<VPL * EPV, false>(a, v, ex);
    }
    store_row<T, EPV, VPL, true>(y + row * n, n, li, tpr, v);
    if (next >= rows) break;
    row = next;
#pragma unroll
    for (int j = 0; j < VPL; ++j) cur[j] = nxt[j];
  }
}

}  // namespace
}  // namespace hmx
