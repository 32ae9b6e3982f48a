// f32 GEMM kernel for gfx950 (v_mfma_f32_32x32x2_f32) and the fixed-order
// split-K reduction shared by every GEMM path.
//
// Same structure as the register-staged bf16 kernel with the f32 MFMA, whose
// operands are one value per lane: LDS keeps each operand in its HBM
// orientation and fragments are gathered with 4-byte (or 16-byte, when
// K-contiguous) reads.
#include "hmx_gemm_common.hpp"

namespace hmx {
namespace {

// f32 kernel.
template <int BM_, int BN_, int BK_>
struct F32Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_;
  // 256 x 256 tiles run 8 waves (2 per SIMD, 2 x 4 over the tile) so that one
  // wave's LDS traffic and barrier hide behind the other's MFMAs.
  static constexpr int NT = BM == 256 ? 512 : 256;
  static constexpr int WAVES_N = NT / 128;
  static constexpr int WM = BM / 2, WN = BN / WAVES_N;
  static constexpr int FM = WM / 32, FN = WN / 32;
};

// LDS image of an f32 operand tile in its HBM orientation: K-contiguous
// `[BR][BK + 4]` or row-contiguous `[BK][BR + 8]` (pads against bank
// conflicts of the fragment reads).
template <int BR, int BK, int NT, int L, bool GUARD>
struct F32Loader {
  static constexpr bool KC = L == L_KCONTIG;
  static constexpr int PITCH = KC ? BK + 4 : BR + 8;
  static constexpr int ELEMS = KC ? BR * PITCH : BK * PITCH;
  static constexpr int ITEMS = BR * BK / 4;
  static constexpr int PER_THREAD = ITEMS / NT;
  static_assert(ITEMS % NT == 0, "tile not divisible among threads");
  uint4 r[PER_THREAD];

  __device__ __forceinline__ void load(const Operand& o, int64_t r0, int64_t k0, int64_t k_end,
                                       int tid) {
    const float* p = (const float*)o.p;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int item = i * NT + tid;
      int64_t row, k;
      if constexpr (KC) {
        row = r0 + item / (BK / 4);
        k = k0 + (item % (BK / 4)) * 4;
      } else {
        k = k0 + item / (BR / 4);
        row = r0 + (item % (BR / 4)) * 4;
      }
      const bool fits = KC ? (row < o.rows && k + 4 <= k_end) : (row + 4 <= o.rows && k < k_end);
      if (!GUARD || (o.vec && fits)) {
        r[i] = *(const uint4*)(p + offset_of<L>(o, row, k));
      } else {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t rr = KC ? row : row + e, kk = KC ? k + e : k;
          v[e] = (rr < o.rows && kk < k_end) ? p[offset_of<L>(o, rr, kk)] : 0.f;
        }
        r[i] = Elem<float>::pack(v);
      }
    }
  }

  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int item = i * NT + tid;
      if constexpr (KC)
        *(uint4*)(lds + (item / (BK / 4)) * PITCH + (item % (BK / 4)) * 4) = r[i];
      else
        *(uint4*)(lds + (item / (BR / 4)) * PITCH + (item % (BR / 4)) * 4) = r[i];
    }
  }

  // The 4 values lane group g feeds MFMAs s = 0..3 of K step k8: K index
  // k8 + 4g + s, row `row` of the tile.
  __device__ __forceinline__ static void frag(const float* lds, int row, int k, float (&v)[4]) {
    if constexpr (KC) {
      const float4 q = *(const float4*)(lds + row * PITCH + k);
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) v[s] = lds[(k + s) * PITCH + row];
    }
  }
};

template <class Cfg, int LAY_A, int LAY_B, bool GUARD>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm_f32_kernel(GemmArgs g) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, NT = Cfg::NT;
  constexpr int FM = Cfg::FM, FN = Cfg::FN;
  using LA = F32Loader<BM, BK, NT, LAY_A, GUARD>;
  using LB = F32Loader<BN, BK, NT, LAY_B, GUARD>;
  __shared__ __attribute__((aligned(16))) float lds[2 * (LA::ELEMS + LB::ELEMS)];
  constexpr int STAGE = LA::ELEMS + LB::ELEMS;

  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, g.xcds, tm, tn);
  const int split = blockIdx.y, batch = blockIdx.z;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t k_begin = (int64_t)split * g.k_chunk;
  const int64_t k_end = min(g.k, k_begin + g.k_chunk);

  Operand a = g.a, b = g.b;
  a.p = (const float*)a.p + batch * g.stride_a;
  b.p = (const float*)b.p + batch * g.stride_b;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / Cfg::WAVES_N, wn = wave % Cfg::WAVES_N;

  LA la;
  LB lb;
  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int ktiles = (int)((k_end - k_begin + BK - 1) / BK);
  if (ktiles > 0) {
    la.load(a, m0, k_begin, k_end, tid);
    lb.load(b, n0, k_begin, k_end, tid);
    la.store(lds, tid);
    lb.store(lds + LA::ELEMS, tid);
  }
  __syncthreads();

  const int frag_row = lane & 31, frag_k = (lane >> 5) * 4;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    // Prefetch the next K tile (the last iteration re-reads its own, in
    // bounds): unconditional, so the staging registers stay registers.
    const int64_t kn = k_begin + (int64_t)min(kt + 1, ktiles - 1) * BK;
    la.load(a, m0, kn, k_end, tid);
    lb.load(b, n0, kn, k_end, tid);
#pragma unroll
    for (int k8 = 0; k8 < BK; k8 += 8) {
      float av[FM][4], bv[FN][4];
#pragma unroll
      for (int i = 0; i < FM; ++i) LA::frag(lds + cur * STAGE, wm * Cfg::WM + i * 32 + frag_row, k8 + frag_k, av[i]);
#pragma unroll
      for (int j = 0; j < FN; ++j) LB::frag(lds + cur * STAGE + LA::ELEMS, wn * Cfg::WN + j * 32 + frag_row, k8 + frag_k, bv[j]);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s], bv[j][s], acc[i][j], 0, 0, 0);
    }
    la.store(lds + (cur ^ 1) * STAGE, tid);
    lb.store(lds + (cur ^ 1) * STAGE + LA::ELEMS, tid);
    __syncthreads();
  }

  if constexpr (BM == 256) {
    // Launched only for split-K partials: identity into f32, no vectors.
    epilogue_direct<FM, FN, Cfg::WM, Cfg::WN, GUARD, ACT_ID, false>(g, split, batch, m0, n0, wm, wn, lane,
                                                                     true, acc);
  } else {
    static_assert(4 * 32 * epi_pitch<Cfg::WN>() <= 2 * STAGE, "epilogue does not fit LDS");
    epilogue<FM, FN, Cfg::WM, Cfg::WN, GUARD>(g, lds, split, batch, m0, n0, wm, wn, wave, lane, acc);
  }
}

// ---------------------------------------------------------------------------
// Split-K reduction: out[b, i, j] = epilogue(sum_s ws[s, b, i, j]) with s in
// increasing order, so the result never depends on scheduling. V consecutive
// columns per thread: 16-byte partial loads and 8/16-byte C stores when rows
// and C keep that alignment (V = 4), else one element (V = 1).
template <int V, bool PROG>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws,
                                                            int splits, int64_t batch,
                                                            GemmArgs g) {
  const int64_t mn = g.m * g.n;
  const int64_t total = batch * mn / V;
  const int64_t split_stride = batch * mn;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t idx = t * V;
    float acc[V];
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] = 0.f;
    for (int sp = 0; sp < splits; ++sp) {
      const float* p = ws + sp * split_stride + idx;
      if constexpr (V == 4) {
        const float4 q = *reinterpret_cast<const float4*>(p);
        acc[0] += q.x;
        acc[1] += q.y;
        acc[2] += q.z;
        acc[3] += q.w;
      } else {
        acc[0] += p[0];
      }
    }
    const int64_t b = idx / mn, rem = idx % mn;
    const int64_t row = rem / g.n, col = rem % g.n;
    float v[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      float bias, scale, shift;
      column_vectors(g, col + e, true, bias, scale, shift);
      v[e] = (acc[e] + bias) * scale + shift;
    }
    activate_all<V, PROG>(g, v);
    const int64_t off = b * g.stride_c + row * g.ldc + col;
    if (g.c_dtype == HMX_DTYPE_BF16) {
      uint16_t* c = (uint16_t*)g.c + off;
      if constexpr (V == 4)
        __builtin_nontemporal_store(
            (uint64_t)pack_bf16x2(v[0], v[1]) | ((uint64_t)pack_bf16x2(v[2], v[3]) << 32), (uint64_t*)c);
      else
        *c = (uint16_t)f32_to_bf16_bits(v[0]);
    } else {
      float* c = (float*)g.c + off;
      if constexpr (V == 4)
        store16_stream(c, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                     __float_as_uint(v[3])));
      else
        *c = v[0];
    }
  }
}

template <class Cfg, int LA, int LB>
void launch_f32(const GemmArgs& g, bool guard, dim3 grid, hipStream_t s) {
  if (guard)
    launch(gemm_f32_kernel<Cfg, LA, LB, true>, grid, Cfg::NT, s, g);
  else
    launch(gemm_f32_kernel<Cfg, LA, LB, false>, grid, Cfg::NT, s, g);
}

template <class Cfg>
void dispatch_f32(const GemmArgs& g, int la, int lb, bool guard, dim3 grid, hipStream_t s) {
  if constexpr (Cfg::BM == 256) {
    if (lb == L_RCONTIG)
      launch_f32<Cfg, L_KCONTIG, L_RCONTIG>(g, guard, grid, s);
    else
      launch_f32<Cfg, L_KCONTIG, L_KCONTIG>(g, guard, grid, s);
  } else if (la == L_KCONTIG) {
    switch (lb) {
      case L_KCONTIG: launch_f32<Cfg, L_KCONTIG, L_KCONTIG>(g, guard, grid, s); break;
      case L_RCONTIG: launch_f32<Cfg, L_KCONTIG, L_RCONTIG>(g, guard, grid, s); break;
      case L_BLOCKED: launch_f32<Cfg, L_KCONTIG, L_BLOCKED>(g, guard, grid, s); break;
      case L_PANELS: launch_f32<Cfg, L_KCONTIG, L_PANELS>(g, guard, grid, s); break;
    }
  } else {
    if (lb == L_KCONTIG)
      launch_f32<Cfg, L_RCONTIG, L_KCONTIG>(g, guard, grid, s);
    else
      launch_f32<Cfg, L_RCONTIG, L_RCONTIG>(g, guard, grid, s);
  }
}

}  // namespace

void launch_gemm_f32(const GemmArgs& g, int tile_bm, int la, int lb, bool guard, dim3 grid,
                     hipStream_t s) {
  if (tile_bm == 256)
    dispatch_f32<F32Cfg<256, 256, 32>>(g, la, lb, guard, grid, s);
  else if (tile_bm == 128)
    dispatch_f32<F32Cfg<128, 128, 32>>(g, la, lb, guard, grid, s);
  else
    dispatch_f32<F32Cfg<64, 64, 32>>(g, la, lb, guard, grid, s);
}

void launch_splitk_reduce(const float* partials, int splits, int64_t batch, const GemmArgs& r,
                          bool vec4, hipStream_t s) {
  const int64_t total = batch * r.m * r.n;
  const bool prog = r.act == HMX_EPI_PROGRAM;
  if (vec4) {
    const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(total / 4, 256), 16384);
    if (prog) launch(splitk_reduce_kernel<4, true>, blocks, 256, s, partials, splits, batch, r);
    else launch(splitk_reduce_kernel<4, false>, blocks, 256, s, partials, splits, batch, r);
  } else {
    const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(total, 256), 16384);
    if (prog) launch(splitk_reduce_kernel<1, true>, blocks, 256, s, partials, splits, batch, r);
    else launch(splitk_reduce_kernel<1, false>, blocks, 256, s, partials, splits, batch, r);
  }
}

}  // namespace hmx
