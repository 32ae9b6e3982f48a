// The 16x16x32 bf16 GEMM kernel body (gemm_bf16_mi16_body), shared by the
// library's instantiations (hmx_gemm_dma.hip) and the kernels hmx_jit.cpp
// compiles at run time with an epilogue compiled in (ACT_JIT).
#pragma once

#include "hmx_gemm_lds.hpp"

namespace hmx {
namespace {

// The eight-wave 64-wide kernel with v_mfma_f32_16x16x32_bf16 in place of
// 32x32x16: whole 256 x 256 tiles, B [N, K], [K, N] or packed (VNNI panels,
// K-major panels, 32 x 32 blocks), K chunks of whole 64-element stages, the register epilogue (identity, ReLU, SiLU). The tiles,
// their swizzles, the loads and the waves' 128 x 64 outputs are those of
// gemm_bf16_dma64_kernel; each wave's outputs are 8 x 4 fragments of 16 x 16.
// A stage is two k-steps of 32 (32 MFMAs each). The GEMM runs at the power
// limit, where what counts is the energy per flop: with random bf16 operands
// a stream of 16x16x32 MFMAs sustains 12 % more than one of 32x32x16 (each
// moves half the accumulator bytes per flop through the register file).
//
// Fragments (lane l, 16-lane group g = l / 16): A (and K-contiguous B) row
// l % 16 of the fragment, K values 8 g .. 8 g + 7 of the k-step (16-byte
// chunk 4 ks + g of the 128-byte tile row, slot chunk ^ swz64(row)); row-major
// B through two transposing reads, of K rows 32 ks + 8 g + 0..3 and + 4..7, lane
// s of each group addressing row + s / 4, columns n + 4 (s % 4) .. + 3 of the
// fragment's 16, so lane j receives column n + j (chunk slot 2 j' + (s % 4) / 2
// ^ bswz(s / 4), byte 8 (s % 2)). The MFMA takes B's fragment first, so an
// accumulator holds row l % 16, columns 4 g .. 4 g + 3 of C.
//
// Slots: 64 MFMAs per stage. The first 12 slots of k-step 0 read k-step 1's
// fragments; at slot 32 the wave waits for its loads of stage t + 1 and its
// reads of stage t, and the barrier publishes t + 1 and frees t; slots 32-51
// issue the 8 loads of stage t + 2 into it and slots 52-63 read stage t + 1's
// k-step 0 fragments.
//
// S stages in LDS (4 for 128 x 128 tiles that run one workgroup per CU):
// the loads issued in stage t are stage t + S's, so S - 1 stages are in
// flight while one is read; the barrier waits only for stage t + 1.
// LDS bytes of the body for these parameters: S stages of the A and B tiles,
// or the staged epilogue's f32 rows where that is larger.
template <int ACT, int BM, int BN, int NW, int S>
constexpr int mi16_lds_bytes() {
  constexpr int stage = BM * 64 * 2 + BN * 64 * 2;
  constexpr int wm = BM / 2, wn = BN / (NW / 2);
  constexpr int epi = NW * (wm / 2) * (wn * 4 + 16);
  return staged_act(ACT) && epi > S * stage ? epi : S * stage;
}

// The body on tile `bid` of g's grid, with `lds` (mi16_lds_bytes, 1 KiB
// aligned) as its LDS; `through`: C is written through to memory (a grid of
// one round).
template <int LB, int ACT, bool BF16, bool RAGGED = false, int BM = 256, int BN = 256, int NW = 8, int S = 2>
__device__ __forceinline__ void gemm_bf16_mi16_body(const GemmArgs& g, uint8_t* lds, int bid, bool through) {
  static_assert(LB == L_KCONTIG || LB == L_RCONTIG || LB == L_VNNI_PANELS || LB == L_PANELS || LB == L_BLOCKED,
                "B [N, K], [K, N], VNNI panels, K-major panels or 32 x 32 blocks");
  static_assert(ACT == ACT_ID || ACT == ACT_RELU || ACT == ACT_SILU || ACT == ACT_JIT || staged_act(ACT),
                "epilogue class");
  static_assert(!staged_act(ACT) || (BM == 256 && BN == 256 && NW == 8 && !RAGGED),
                "other epilogues: whole 256 x 256 tiles");
  static_assert(!RAGGED || LB == L_KCONTIG || LB == L_RCONTIG, "ragged tiles: B [N, K] or [K, N]");
  // Tiles: 256 x 256 with eight waves of 128 x 64; 128 x 128 with four of
  // 64 x 64; 256 x 128 with eight of 128 x 32.
  static_assert((BM == 256 && BN == 256 && NW == 8) || (BM == 128 && BN == 128 && NW == 4) ||
                    (BM == 256 && BN == 128 && NW == 8),
                "256 x 256 (8 waves), 128 x 128 (4 waves) or 256 x 128 (8 waves)");
  static_assert(BN == 256 || LB == L_KCONTIG || LB == L_RCONTIG, "packed B: 256-column tiles");
  static_assert(S == 2 || (S == 4 && BM == 128 && BN == 128 && !staged_act(ACT)), "stages: 2, or 4 of 128 x 128");
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  // Packed B as in gemm_bf16_dma64_kernel: K-major panels and 32 x 32 blocks
  // land in LDS as the row-major [64 k][256 n] tile (BT), VNNI panels as
  // copied.
  constexpr bool BPK = LB == L_PANELS || LB == L_BLOCKED;
  constexpr bool BT = LB == L_RCONTIG || BPK;
  constexpr bool VN = LB == L_VNNI_PANELS;
  constexpr int BK = 64;
  constexpr int ROWB = BK * 2, NROWB = BN * 2;
  constexpr int A_BYTES = BM * ROWB;            // 32 KiB (16 KiB for 128-row tiles)
  constexpr int STAGE = A_BYTES + BN * BK * 2;  // 64 KiB (32 or 48 KiB)
  constexpr int WM = BM / 2, WN = BN / (NW / 2), FM = WM / 16, FN = WN / 16;
  constexpr int LA = BM / 8 / NW, LBN = BN / 8 / NW, LOADS = LA + LBN;  // 4 + 4 (8 + 4 for 256 x 128)
  constexpr int NS = FM * FN, SLOTS = 2 * NS, NF = FM + FN;            // 32, 64, 12 (16, 32, 8)
  constexpr int BAR = NS, LOAD_END = SLOTS - NF;                         // 32, 52 (16, 24)
  // ACT_ANY stages each wave's 64-row halves as f32, rows of WN * 4 + 16
  // bytes: 8 x 64 x 272 bytes, a little more than the stages.
  constexpr int LDS_BYTES = mi16_lds_bytes<ACT, BM, BN, NW, S>();
  static_assert(LDS_BYTES <= 160 * 1024, "LDS");

  int tm, tn;
  tile_coords(bid, g.tiles_m, g.tiles_n, g.xcds, tm, tn);
  const int split = blockIdx.y, batch = blockIdx.z;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t k_begin = (int64_t)split * g.k_chunk;
  const int64_t k_end = min(g.k, k_begin + g.k_chunk);
  const int ktiles = (int)((k_end - k_begin) / BK);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / (NW / 2), wn = wave % (NW / 2);

  const i32x4_t srd_a = make_srd((const uint16_t*)g.a.p + batch * g.stride_a, g.a.bytes);
  const i32x4_t srd_b = make_srd((const uint16_t*)g.b.p + batch * g.stride_b, g.b.bytes);
  // Loads, as gemm_bf16_dma64_kernel with eight waves: wave w copies tile rows
  // 32 w .. 32 w + 31 of A (and of K-contiguous B), 8 rows per 1 KiB load, or
  // K rows 8 w .. 8 w + 7 of row-major B in pairs.
  const int rr = lane >> 3, slot = lane & 7;
  auto kc_voff = [&](int64_t ld, int par) {
    return (int32_t)((rr * ld + (slot ^ ((rr >> 1) | (par << 2))) * 8) * 2);
  };
  const int32_t voff_a0 = kc_voff(g.a.ld, 0), voff_a1 = kc_voff(g.a.ld, 1);
  // RAGGED (M or N not whole tiles), as gemm_bf16_dma64_kernel: a buffer
  // load's scalar offset is not range-checked, so each lane's whole row of A
  // (of K-contiguous B) sits in its vector offset, clamped to the last row,
  // row-major B's columns clamped to the last 8-column chunk, and the scalar
  // offset holds only the K position. The duplicated rows and columns reach
  // only outputs that are never stored.
  auto kc_voff_clamped = [&](int64_t ld, int64_t row, int64_t rows, int par) {
    return (int32_t)((min(row, rows - 1) * ld + (slot ^ ((rr >> 1) | (par << 2))) * 8) * 2);
  };
  int32_t va[RAGGED ? LA : 1], vb[RAGGED && !BT ? LBN : 1];
  if constexpr (RAGGED) {
#pragma unroll
    for (int q = 0; q < LA; ++q) va[q] = kc_voff_clamped(g.a.ld, m0 + wave * (BM / NW) + q * 8 + rr, g.m, q & 1);
    if constexpr (!BT) {
#pragma unroll
      for (int q = 0; q < LBN; ++q)
        vb[q] = kc_voff_clamped(g.b.ld, n0 + wave * (BN / NW) + q * 8 + rr, g.n, q & 1);
    }
  }
  const int32_t soff_a = (int32_t)((m0 + wave * (BM / NW)) * g.a.ld * 2);
  const int32_t blk_a = (int32_t)(8 * g.a.ld * 2);
  int32_t voff_b0, voff_b1, soff_b, blk_b;
  int32_t vn_off[VN ? LBN : 1];
  const int64_t P = g.b.panel;
  if constexpr (VN) {
    // The stage lands re-laid in 16-byte pieces (4 columns of one K pair) so
    // that one fragment read of the 16 x 16 x 32 MFMA is 256 consecutive
    // bytes: slabs of 4 KiB, one per K pair kp = 16 ks + 4 f + i (i, ks
    // outer), each holding the tile's 16 groups of 16 columns as 256-byte
    // lines [f 4][16 columns][K pair]. 1 KiB load b (of the stage's 32) fills
    // slab (ks, i) = (b / 16, b / 4 % 4), groups 4 (b % 4) .. + 3; lane l
    // takes group 4 (b % 4) + l / 16, f = l / 4 % 4, columns 4 (l % 4) .. + 3,
    // i.e. K-pair row 16 ks + 4 f + i of tile columns 64 (b % 4) + lam,
    // lam = 16 (l / 16) + 4 (l % 4). Every load still reads 8 whole 128-byte
    // rows. A lane's part of the offset is its K-pair row f and column lam
    // (a 32-column panel boundary falls inside lam for P = 32); the load's
    // part is the slab and the 64-column group. P is a multiple of 32 that
    // divides 256, or a multiple of 256, so (n0 + 64 (b % 4)) % P + lam stays in
    // one panel for P > 32.
    const int f = (lane >> 2) & 3, lam = 16 * (lane >> 4) + 4 * (lane & 3);
    voff_b0 = voff_b1 = (int32_t)(f * 16 * P + (lam / P) * (g.b.kpad / 2) * 4 * P + (lam % P) * 4);
    soff_b = blk_b = 0;
#pragma unroll
    for (int q = 0; q < LBN; ++q) {
      const int b = wave * LBN + q, ks = b >> 4, i = (b >> 2) & 3;
      const int64_t col = n0 + 64 * (b & 3);
      vn_off[q] = (int32_t)((16 * ks + i) * 4 * P + (col / P) * (g.b.kpad / 2) * 4 * P + (col % P) * 4);
    }
  } else if constexpr (BPK) {
    // Element (k, n) at col(n) + row(k); a lane's 8 columns stay in one panel
    // or block, the lane offset holds col(n) and the row within the K pair.
    // Rows 8 w .. 8 w + 7: bit 3 of the row is the wave's parity.
    const int r = lane >> 5, c = (lane & 31) ^ (((wave * (64 / NW)) >> 2) & 2);
    auto col = [&](int64_t n) -> int64_t {
      if constexpr (LB == L_PANELS) return (n / P) * g.b.kpad * P + n % P;
      else return (n >> 5) * (g.b.kpad >> 5) * 1024 + (n & 31);
    };
    const int64_t rs = LB == L_PANELS ? P : 32;
    voff_b0 = (int32_t)((col(n0 + (c ^ swz_n(r)) * 8) + r * rs) * 2);
    voff_b1 = (int32_t)((col(n0 + (c ^ swz_n(r + 2)) * 8) + r * rs) * 2);
    soff_b = blk_b = 0;
  } else if constexpr (BT && BN == 128) {
    // 256-byte rows: a 1 KiB load is 4 K rows, lane l filling slot l % 16 of
    // row l / 16; row k % 4 == l / 16 for every load. Bit 3 of the row flips
    // chunk bit 1 (bswz): voff_b0 for rows with it clear, voff_b1 set.
    const int r = lane >> 4, c = lane & 15;
    const int h = ((wave * (64 / NW)) >> 2) & 2;  // bit 3 of the wave's first row, as chunk bit 1
    if constexpr (RAGGED) {
      const int64_t last = ((g.n - 1) >> 3) << 3;  // the last 8-column chunk
      voff_b0 = (int32_t)((r * g.b.ld + min(n0 + (c ^ swz_n(r) ^ h) * 8, last)) * 2);
      voff_b1 = (int32_t)((r * g.b.ld + min(n0 + (c ^ swz_n(r) ^ h ^ 2) * 8, last)) * 2);
      soff_b = (int32_t)(wave * (64 / NW) * g.b.ld * 2);
    } else {
      voff_b0 = (int32_t)((r * g.b.ld + (c ^ swz_n(r) ^ h) * 8) * 2);
      voff_b1 = (int32_t)((r * g.b.ld + (c ^ swz_n(r) ^ h ^ 2) * 8) * 2);
      soff_b = (int32_t)((wave * (64 / NW) * g.b.ld + n0) * 2);
    }
    blk_b = (int32_t)(4 * g.b.ld * 2);
  } else if constexpr (BT) {
    // Rows 8 w .. 8 w + 7 (eight waves): bit 3 of the row is the wave's
    // parity, folded into the chunk (bswz).
    const int r = lane >> 5, c = (lane & 31) ^ (((wave * (64 / NW)) >> 2) & 2);
    if constexpr (RAGGED) {
      const int64_t last = ((g.n - 1) >> 3) << 3;  // the last 8-column chunk
      voff_b0 = (int32_t)((r * g.b.ld + min(n0 + (c ^ swz_n(r)) * 8, last)) * 2);
      voff_b1 = (int32_t)((r * g.b.ld + min(n0 + (c ^ swz_n(r + 2)) * 8, last)) * 2);
      soff_b = (int32_t)(wave * (64 / NW) * g.b.ld * 2);
    } else {
      voff_b0 = (int32_t)((r * g.b.ld + (c ^ swz_n(r)) * 8) * 2);
      voff_b1 = (int32_t)((r * g.b.ld + (c ^ swz_n(r + 2)) * 8) * 2);
      soff_b = (int32_t)((wave * (64 / NW) * g.b.ld + n0) * 2);
    }
    blk_b = (int32_t)(2 * g.b.ld * 2);
  } else {
    voff_b0 = kc_voff(g.b.ld, 0);
    voff_b1 = kc_voff(g.b.ld, 1);
    soff_b = (int32_t)((n0 + wave * (BN / NW)) * g.b.ld * 2);
    blk_b = (int32_t)(8 * g.b.ld * 2);
  }
  const uint32_t lds_w = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + wave * LA * 1024;
  const uint32_t lds_wb = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + A_BYTES + wave * LBN * 1024;
  auto dma = [&](int t, int q) {
    const int64_t k0 = k_begin + (int64_t)min(t, ktiles - 1) * BK;
    const uint32_t st = lds_w + (uint32_t)((t & (S - 1)) * STAGE);
    const uint32_t sb = lds_wb + (uint32_t)((t & (S - 1)) * STAGE);
    if (q < LA) {
      if constexpr (RAGGED)
        lds_dma16(srd_a, va[q], (int32_t)(k0 * 2), st + q * 1024);
      else
        lds_dma16(srd_a, (q & 1) ? voff_a1 : voff_a0, soff_a + q * blk_a + (int32_t)(k0 * 2), st + q * 1024);
    } else if constexpr (VN) {
      const int qb = q - LA;
      lds_dma16(srd_b, voff_b0, vn_off[qb] + (int32_t)((k0 / 2) * 4 * P), sb + qb * 1024);
    } else if constexpr (BPK) {
      const int qb = q - LA;
      const int64_t kr = k0 + wave * (64 / NW) + 2 * qb;  // even
      const int64_t row = LB == L_PANELS ? kr * P : (kr >> 5) * 1024 + (kr & 31) * 32;
      lds_dma16(srd_b, (qb & 1) ? voff_b1 : voff_b0, (int32_t)(row * 2), sb + qb * 1024);
    } else if constexpr (RAGGED && !BT) {
      const int qb = q - LA;
      lds_dma16(srd_b, vb[qb], (int32_t)(k0 * 2), sb + qb * 1024);
    } else {
      const int qb = q - LA;
      const int32_t kb = BT ? (int32_t)(k0 * g.b.ld * 2) : (int32_t)(k0 * 2);
      // 256-byte B rows: load qb covers rows 4 qb .. 4 qb + 3 of the wave's,
      // bit 3 of which is that of qb >> 1.
      const bool hi = BT && BN == 128 ? (qb >> 1) & 1 : qb & 1;
      lds_dma16(srd_b, hi ? voff_b1 : voff_b0, soff_b + qb * blk_b + kb, sb + qb * 1024);
    }
  };

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int frow = lane & 15, fg = lane >> 4, fswz = swz64(frow);
  const uint8_t* a_frag = lds + (wm * WM + frow) * ROWB;
  const uint8_t* b_frag = lds + A_BYTES + (wn * WN + frow) * ROWB;
  int b_tr[FN];
  {
    const int sl = lane & 15;
#pragma unroll
    for (int j = 0; j < FN; ++j)
      b_tr[j] = A_BYTES + (8 * fg + (sl >> 2)) * NROWB +
                ((wn * (WN / 8) + 2 * j + ((sl & 3) >> 1)) ^ bswz(8 * fg + (sl >> 2))) * 16 + 8 * (sl & 1);
  }
  auto a_read = [&](int stage, int ks, int i) -> bf16x8_t {
    return *(const bf16x8_t*)(a_frag + stage * STAGE + i * 16 * ROWB + ((4 * ks + fg) ^ fswz) * 16);
  };
  // VNNI B: column n = wn * 64 + 16 j + lane % 16 needs K pairs
  // 16 ks + 4 (lane / 16) + i, i = 0 .. 3 (K values 32 ks + 8 (lane / 16)
  // .. + 7, the MFMA's operand): one 4-byte read per slab, lane l at byte
  // 4 (l % 16) of f = l / 16's 64 bytes of the column group's line.
  constexpr int VSLAB = BN * 16;  // 4 KiB: one K pair of each tile column
  const int b_vn = A_BYTES + (wn * (WN / 16)) * 256 + fg * 64 + frow * 4;
  auto b_read = [&](int stage, int ks, int j) -> bf16x8_t {
    if constexpr (VN) {
      const uint8_t* p = lds + stage * STAGE + b_vn + j * 256 + ks * 4 * VSLAB;
      const uint4 v = make_uint4(*(const uint32_t*)p, *(const uint32_t*)(p + VSLAB),
                                 *(const uint32_t*)(p + 2 * VSLAB), *(const uint32_t*)(p + 3 * VSLAB));
      return __builtin_bit_cast(bf16x8_t, v);
    } else if constexpr (BT) {
      const uint8_t* p = lds + stage * STAGE + b_tr[j] + 32 * ks * NROWB;
      return __builtin_shufflevector(lds_read_tr(p), lds_read_tr(p + 4 * NROWB), 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      return *(const bf16x8_t*)(b_frag + stage * STAGE + j * 16 * ROWB + ((4 * ks + fg) ^ fswz) * 16);
    }
  };

  // The host launches this kernel only with at least one K stage per split.
  bf16x8_t fa[2][FM], fb[2][FN];
#pragma unroll
  for (int u = 0; u < S; ++u)
#pragma unroll
    for (int q = 0; q < LOADS; ++q) dma(u, q);
  wait_vmem<LOADS * (S - 1)>();  // stage 0 landed
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = a_read(0, 0, i);
#pragma unroll
  for (int j = 0; j < FN; ++j) fb[0][j] = b_read(0, 0, j);

  // One K stage. LOADS_C: the stage issues stage t + S's loads. With two
  // stages the last two issue none (the barrier's wait is for every load,
  // vmcnt 0), in a copy of the stage without them rather than behind a branch
  // per load; with four the barrier counts on S - 2 stages of loads behind
  // the next, which clamped reloads of the last stage keep.
  auto stage = [&](int t, auto loads_c) {
    constexpr bool LOADS_C = decltype(loads_c)::value;
    const int cur = t & (S - 1), nxt = (t + 1) & (S - 1);
#pragma unroll
    for (int x = 0; x < SLOTS; ++x) {
      __builtin_amdgcn_sched_barrier(0);
      const int ks = x / NS, sub = x % NS;
      if (x == BAR)
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(LOADS * (S - 2)) : "memory");
      if (ks == 0 && sub < NF) {
        if (sub < FM) fa[1][sub] = a_read(cur, 1, sub);
        else fb[1][sub - FM] = b_read(cur, 1, sub - FM);
      }
      // The stage's loads, spread over the slots from the barrier to the
      // next stage's fragment reads.
#pragma unroll
      for (int q = (x - BAR) * LOADS / (LOAD_END - BAR); q < (x + 1 - BAR) * LOADS / (LOAD_END - BAR); ++q)
        if (LOADS_C && x >= BAR && x < LOAD_END) dma(t + S, q);
      if (x >= SLOTS - NF) {
        const int f = x - (SLOTS - NF);
        if (f < FM) fa[0][f] = a_read(nxt, 0, f);
        else fb[0][f - FM] = b_read(nxt, 0, f - FM);
      }
      const int i = sub / FN, j = sub % FN;
      // B's fragment first: the product is C^T's fragment, so each lane ends
      // with four adjacent columns of one row of C.
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[ks][j], fa[ks][i], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (S == 2) {
    int t = 0;
    for (; t < ktiles - S; ++t) stage(t, std::true_type{});
    for (; t < ktiles; ++t) stage(t, std::false_type{});
  } else {
    for (int t = 0; t < ktiles; ++t) stage(t, std::true_type{});
  }
  wait_vmem<0>();  // no load into LDS outlives the loop

  // Epilogue. Lane l holds row l % 16 of each fragment, columns
  // 4 (l / 16) .. + 3 (the operands went in B first): bias, scale, shift,
  // activation, one rounding. Without bias, scale and shift (the common
  // case) the affine step is skipped; it would only turn -0 into +0.
  const int64_t off = split * g.stride_split + batch * g.stride_c;
  const bool affine = g.bias || g.scale || g.shift;
  // The lane's four columns of fragment column j (tile coordinates).
  auto col4_of = [&](int j) { return wn * WN + j * 16 + 4 * fg; };
  // Bias, scale and shift of the lane's four columns of fragment column j
  // (columns past N: identity values, for ragged tiles).
  auto vectors4 = [&](int j, float (&cb)[4], float (&cs)[4], float (&ch)[4]) {
    column_vectors4(g, n0 + col4_of(j), g.n, cb, cs, ch);
  };
  // `through` (the grid is one round, a workgroup per CU at most): C is
  // written through to memory, so the kernel ends with few dirty L2 lines to
  // write back (an f32 C of 4096 x 4096 finishes 5-6% sooner). With more
  // rounds the streaming stores are kept: a workgroup retires only once its
  // stores are acknowledged, and written-through stores are acknowledged
  // later, which delays the next round's workgroups (~5% slower at 1376
  // tiles).
  auto store_c = [&](void* p, const uint4& v) {
    if (through) store16_through(p, v);
    else store16_stream(p, v);
  };
  if constexpr (staged_act(ACT)) {
    // Any other named activation, or an epilogue program: each wave stages
    // its own 128 x 64 outputs as f32 in its own LDS region, 64 rows at a
    // time (rows padded by 16 bytes; a lane writes its four columns of a
    // fragment row as one 16-byte store, and the 16 rows of one write meet
    // distinct banks), and finishes them in runs of 8 columns -- bias,
    // scale, shift, the activation or program, one rounding -- in a loop that
    // is not unrolled, so the interpreter is emitted once per half, storing
    // each run with a 16-byte write. Half by half, the accumulators it has
    // stored are no longer live, which leaves the interpreter its registers.
    constexpr int PW = WN * 4 + 16;  // f32 row pitch of a wave's region
    static_assert(NW * (WM / 2) * PW <= LDS_BYTES, "the waves' regions fit");
    uint8_t* region = lds + wave * (WM / 2) * PW;
    constexpr int RUNS = WN / 8;  // runs of 8 columns per row
    static_assert(64 % RUNS == 0, "a lane's run is the same in every step");
    // The lane's 8 columns are the same in every step below: their bias,
    // scale and shift are loaded once (inside the loop the stores to C keep
    // the compiler from hoisting the loads).
    const int c8 = (lane % RUNS) * 8;
    const int64_t col = n0 + wn * WN + c8;
    float cb[8], cs[8], ch[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) column_vectors(g, col + e, true, cb[e], cs[e], ch[e]);
    __syncthreads();  // every wave is done with the stages
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      with_index<2>(q, [&](auto q_c) {
        constexpr int Q = decltype(q_c)::value;
#pragma unroll
        for (int i = Q * (FM / 2); i < (Q + 1) * (FM / 2); ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            *(f32x4_t*)(region + ((i - Q * (FM / 2)) * 16 + frow) * PW + (j * 16 + 4 * fg) * 4) = acc[i][j];
      });
#pragma unroll 1
      for (int it = 0; it < (WM / 2) * RUNS / 64; ++it) {
        const int r = (it * 64 + lane) / RUNS;
        const float4 lo = *(const float4*)(region + r * PW + c8 * 4);
        const float4 hi = *(const float4*)(region + r * PW + c8 * 4 + 16);
        float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (v[e] + cb[e]) * cs[e] + ch[e];
        activate_all<8, ACT == ACT_PROG>(g, v);
        const int64_t row = m0 + wm * WM + q * (WM / 2) + r;
        if constexpr (BF16) {
          store_c((uint16_t*)g.c + off + row * g.ldc + col, Elem<uint16_t>::pack(v));
        } else {
          float* cp = (float*)g.c + off + row * g.ldc + col;
          store_c(cp, Elem<float>::pack(v));
          store_c(cp + 4, Elem<float>::pack(v + 4));
        }
      }
    }
  } else if constexpr (BF16) {
    // bf16 C leaves through LDS, each wave through its own region of the
    // stage buffers (free once every wave is done with the last stage): its
    // WM x WN outputs as rows of PB = 2 WN bytes. Fragment row block by
    // block, a lane writes its four columns of a row as one 8-byte word, then
    // the wave reads the block's 16 rows back as 16-byte chunks of whole row
    // pieces (one 128-byte line each for 256-column tiles) and stores them:
    // no wave waits for another, and a block's stores overlap the next
    // block's writes. Written straight from the fragments, each store would
    // cover 32-byte pieces of 16 rows. Chunk c of region row r sits in slot
    // c ^ ((r / RPB) % CPW), RPB rows per 256 bytes, so the 16 rows x 32 bytes
    // of one write and the rows of one read meet distinct banks.
    constexpr int PB = WN * 2, CPW = PB / 16, RPB = 256 / PB, RPI = 64 / CPW;
    static_assert(NW * WM * PB <= LDS_BYTES && RPB * PB == 256 && 16 % RPI == 0, "bf16 C regions");
    __syncthreads();
    uint8_t* region = lds + wave * (WM * PB);
    auto slot = [](int r, int c) { return r * PB + ((c ^ ((r / RPB) % CPW)) << 4); };
    uint16_t* c = (uint16_t*)g.c + off;
    const int64_t row0 = m0 + wm * WM, col0 = n0 + wn * WN;
    auto run = [&](auto&& finish) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = i * 16 + frow;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = finish(acc[i][j][e], j, e);
          *(uint2*)(region + slot(r, 2 * j + (fg >> 1)) + (fg & 1) * 8) =
              make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        }
        // The block's rows are read back by other lanes of this wave: the
        // wave's LDS accesses run in order, and the compiler keeps the reads
        // after the writes.
        asm volatile("" ::: "memory");
#pragma unroll
        for (int p = 0; p < 16 / RPI; ++p) {
          const int rr = i * 16 + p * RPI + lane / CPW, ch = lane % CPW;
          const uint4 v = *(const uint4*)(region + slot(rr, ch));
          const int64_t row = row0 + rr, col = col0 + ch * 8;
          if constexpr (RAGGED) {
            // Rows past M are not stored; the chunk across N is stored
            // element by element.
            if (row < g.m) {
              if (col + 8 <= g.n) {
                store_c(c + row * g.ldc + col, v);
              } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                  if (col + e < g.n) c[row * g.ldc + col + e] = (uint16_t)(dw(v, e >> 1) >> (16 * (e & 1)));
              }
            }
          } else {
            store_c(c + row * g.ldc + col, v);
          }
        }
      }
    };
    if (affine) {
      float vb[FN][4], vs[FN][4], vh[FN][4];
#pragma unroll
      for (int j = 0; j < FN; ++j) vectors4(j, vb[j], vs[j], vh[j]);
      run([&](float a, int j, int e) { return activate<ACT>((a + vb[j][e]) * vs[j][e] + vh[j][e]); });
    } else {
      run([](float a, int, int) { return activate<ACT>(a); });
    }
  } else {
    // f32 C straight from the fragments: a lane's four columns of a row are
    // one 16-byte store where C's rows allow it (16-byte aligned, whole), else
    // four 4-byte stores.
    float* c = (float*)g.c + off;
    const bool vec = ((((uintptr_t)g.c) & 15) == 0) && g.ldc % 4 == 0 && g.stride_c % 4 == 0 &&
                     g.stride_split % 4 == 0;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = n0 + col4_of(j);
      float cb[4], cs[4], ch[4];
      vectors4(j, cb, cs, ch);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int64_t row = m0 + wm * WM + i * 16 + frow;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = activate<ACT>((acc[i][j][e] + cb[e]) * cs[e] + ch[e]);
        float* cp = c + row * g.ldc + col;
        if ((!RAGGED || (row < g.m && col + 4 <= g.n)) && vec) {
          store_c(cp, Elem<float>::pack(v));
        } else if (!RAGGED || row < g.m) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (!RAGGED || col + e < g.n) store_c32(cp + e, __float_as_uint(v[e]));
        }
      }
    }
  }
}

// The body as a kernel of its own: the workgroup's tile is blockIdx.x, and C
// is written through when the grid is one round.
template <int LB, int ACT, bool BF16, bool RAGGED = false, int BM = 256, int BN = 256, int NW = 8, int S = 2>
__device__ __forceinline__ void gemm_bf16_mi16_body(const GemmArgs& g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[mi16_lds_bytes<ACT, BM, BN, NW, S>()];
  gemm_bf16_mi16_body<LB, ACT, BF16, RAGGED, BM, BN, NW, S>(
      g, lds, (int)blockIdx.x, gridDim.x * gridDim.y * gridDim.z <= (unsigned)g.cus);
}

}  // namespace
}  // namespace hmx
