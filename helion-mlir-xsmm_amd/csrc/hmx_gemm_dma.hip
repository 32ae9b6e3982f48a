// Direct-to-LDS bf16 GEMM kernels for gfx950 (v_mfma_f32_32x32x16_bf16):
// whole 256 x 256 tiles of row-major A and a B that is either K-contiguous
// ([N, K]) or row-major ([K, N]). Operand tiles go from memory straight into
// LDS (`buffer_load_dwordx4 ... lds`), with no VGPR staging and no LDS write
// instructions. Two variants: 64-wide K stages (two stages of 64 KiB, below)
// for K chunks of whole 64-element stages, and 32-wide K tiles (four stages
// of 32 KiB, three in flight) otherwise.
//
// LDS tiles are unpadded: one such load fills 1 KiB of LDS contiguously
// (lane l at byte 16 l), so bank conflicts are avoided by XOR-swizzling
// 16-byte chunks instead -- the lane that fills slot c of tile row r fetches
// global chunk c ^ swz(r).
//  * A, and K-contiguous B: [256 rows][32 k], 64-byte rows (4 chunks),
//    swz_k(r) = ((r >> 1) & 3) ^ ((r >> 3) & 1). A fragment read (16 bytes:
//    row lane % 32, chunk 2 ks + lane / 32) then meets distinct banks whether
//    LDS serves 8 or 16 lanes per cycle.
//  * row-major B: [32 k][256 n], 512-byte rows (32 chunks),
//    swz_n(r) = ((r & 3) << 1) ^ ((r & 3) << 2). Fragments come from
//    ds_read_b64_tr_b16, which transposes within each group of 16 lanes:
//    lane j receives, as its element e, element j % 4 of the 8 bytes lane
//    4 e + j / 4 addressed. Lane s of a group addresses row k0 + s / 4 at
//    columns n0 + 4 (s % 4) .. + 3, so lane j ends with B[k0 .. k0 + 3][n0 + j],
//    the MFMA's K-ordered operand; two such reads make the 8-value operand.
//    The 4 rows x 2 (16 lanes) or 4 (32 lanes) chunks touched per pass land
//    on distinct banks.
//
// These loads and their waits are inline assembly: the compiler would
// otherwise wait for every outstanding LDS load (vmcnt(0)) before any LDS
// read, which leaves nothing in flight. Loads complete in issue order, so the
// compiler's own waits for other memory operations stay correct.
#include <cstdlib>

#include "hmx_gemm_lds.hpp"
#include "hmx_gemm_mi16.hpp"

namespace hmx {
namespace {


// One instantiation per B orientation, register-epilogue class and C dtype:
// a single straight-line epilogue keeps the accumulators out of scratch.
template <int LB, int ACT, bool BF16>
__global__ __launch_bounds__(256, 1) void gemm_bf16_dma_kernel(GemmArgs g) {
  constexpr bool BT = LB == L_RCONTIG;             // B row-major [K, N]
  constexpr int BM = 256, BN = 256, BK = 32, S = 4;
  constexpr int ROWB = BK * 2;                     // bytes per K-contiguous tile row
  constexpr int NROWB = BN * 2;                    // bytes per row-major B tile row
  constexpr int A_BYTES = BM * ROWB;               // 16 KiB
  constexpr int STAGE = A_BYTES + BN * BK * 2;     // 32 KiB
  constexpr int FM = 4, FN = 4, WM = 128, WN = 128;
  constexpr int LOADS = 8;                         // DMA instructions per wave per tile
  __shared__ __attribute__((aligned(1024))) uint8_t lds[S * STAGE];

  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, g.xcds, tm, tn);
  const int split = blockIdx.y, batch = blockIdx.z;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t k_begin = (int64_t)split * g.k_chunk;
  const int64_t k_end = min(g.k, k_begin + g.k_chunk);
  const int ktiles = (int)((k_end - k_begin) / BK);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  const i32x4_t srd_a = make_srd((const uint16_t*)g.a.p + batch * g.stride_a, g.a.bytes);
  const i32x4_t srd_b = make_srd((const uint16_t*)g.b.p + batch * g.stride_b, g.b.bytes);
  // Wave w loads 16-row blocks 4w .. 4w + 3 of the A tile: lane l fills slot
  // l % 4 of block row l / 4. Byte offsets below 2^31: the operands' byte
  // ranges are.
  const int drow = lane >> 2;
  const int32_t voff_a = (int32_t)((drow * g.a.ld + ((lane & 3) ^ swz_k(drow)) * 8) * 2);
  const int32_t soff_a = (int32_t)((m0 + wave * 64) * g.a.ld * 2);
  const int32_t blk_a = (int32_t)(16 * g.a.ld * 2);
  // B: K-contiguous as A; row-major in pairs of rows 8w + 2q, 8w + 2q + 1
  // (q < 4), lane l filling slot l % 32 of row l / 32 of the pair.
  int32_t voff_b0, voff_b1, soff_b, blk_b;
  if constexpr (BT) {
    const int r = lane >> 5, c = lane & 31;
    voff_b0 = (int32_t)((r * g.b.ld + (c ^ swz_n(r)) * 8) * 2);      // even q
    voff_b1 = (int32_t)((r * g.b.ld + (c ^ swz_n(r + 2)) * 8) * 2);  // odd q
    soff_b = (int32_t)((wave * 8 * g.b.ld + n0) * 2);
    blk_b = (int32_t)(2 * g.b.ld * 2);
  } else {
    voff_b0 = voff_b1 = (int32_t)((drow * g.b.ld + ((lane & 3) ^ swz_k(drow)) * 8) * 2);
    soff_b = (int32_t)((n0 + wave * 64) * g.b.ld * 2);
    blk_b = (int32_t)(16 * g.b.ld * 2);
  }
  const uint32_t lds_w = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + wave * 4 * 1024;

  // DMA q (< 8) of tile t: A blocks for q < 4, then B.
  auto dma = [&](int t, int q) {
    const int64_t k0 = k_begin + (int64_t)min(t, ktiles - 1) * BK;
    const uint32_t st = lds_w + (uint32_t)((t % S) * STAGE);
    if (q < 4) {
      lds_dma16(srd_a, voff_a, soff_a + q * blk_a + (int32_t)(k0 * 2), st + q * 1024);
    } else {
      const int32_t kb = BT ? (int32_t)(k0 * g.b.ld * 2) : (int32_t)(k0 * 2);
      lds_dma16(srd_b, (q & 1) ? voff_b1 : voff_b0, soff_b + (q - 4) * blk_b + kb,
                st + A_BYTES + (q - 4) * 1024);
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment reads. A (and K-contiguous B): row lane % 32 of the fragment,
  // chunk 2 ks + lane / 32.
  const int frow = lane & 31, fk = lane >> 5, fswz = swz_k(frow);
  const uint8_t* a_frag = lds + (wm * WM + frow) * ROWB;
  const uint8_t* b_frag = lds + A_BYTES + (wn * WN + frow) * ROWB;
  // Row-major B: lane s of 16-lane group gi addresses row 8 (gi / 2) + s / 4
  // (+ 16 ks, + 4 for the second read) and the chunk holding columns
  // wn * 128 + 32 j + 16 (gi % 2) + 4 (s % 4).
  int b_tr[FN];
  {
    const int gi = lane >> 4, sl = lane & 15;
    const int v = (2 * (gi & 1) + ((sl & 3) >> 1)) ^ swz_n(sl >> 2);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      b_tr[j] = A_BYTES + (8 * (gi >> 1) + (sl >> 2)) * NROWB + (wn * 16 + ((4 * j) ^ v)) * 16 + 8 * (sl & 1);
  }
  auto a_read = [&](int stage, int ks, int i) -> bf16x8_t {
    return *(const bf16x8_t*)(a_frag + stage * STAGE + i * 32 * ROWB + ((2 * ks + fk) ^ fswz) * 16);
  };
  auto b_read = [&](int stage, int ks, int j) -> bf16x8_t {
    if constexpr (BT) {
      const uint8_t* p = lds + stage * STAGE + b_tr[j] + 16 * ks * NROWB;
      return __builtin_shufflevector(lds_read_tr(p), lds_read_tr(p + 4 * NROWB), 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      return *(const bf16x8_t*)(b_frag + stage * STAGE + j * 32 * ROWB + ((2 * ks + fk) ^ fswz) * 16);
    }
  };

  // The host launches this kernel only with at least one K tile per split.
  bf16x8_t a0[FM], b0[FN], a1[FM], b1[FN];
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int q = 0; q < LOADS; ++q) dma(t, q);
  wait_vmem<2 * LOADS>();  // tile 0 landed
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FM; ++i) a0[i] = a_read(0, 0, i);
#pragma unroll
  for (int j = 0; j < FN; ++j) b0[j] = b_read(0, 0, j);

  for (int t = 0; t < ktiles; ++t) {
    // Tiles t + 1 and t + 2 are in flight: wait for t + 1, then the barrier
    // publishes it and frees stage (t + 3) % S (last read in step t - 1).
    // The barrier carries no LDS fence: every LDS read of the freed stage
    // was consumed by an MFMA of step t - 1 before it.
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(LOADS) : "memory");
    const int cur = t % S, nxt = t + 1 < ktiles ? (t + 1) % S : cur;
    // 32 MFMA slots per step, each paired with at most one other memory
    // operation: slots 0-7 read k-step 1's fragments, slots 8-15 issue the
    // DMA of tile t + 3, slots 16-23 read the next tile's k-step 0 fragments
    // (a quarter step ahead of the barrier that follows).
#pragma unroll
    for (int x = 0; x < 32; ++x) {
      __builtin_amdgcn_sched_barrier(0);
      const int f = x & 7;
      if (x < 8) {
        if (f < 4) a1[f] = a_read(cur, 1, f);
        else b1[f - 4] = b_read(cur, 1, f - 4);
      } else if (x < 16) {
        dma(t + 3, f);
      } else if (x < 24) {
        if (f < 4) a0[f] = a_read(nxt, 0, f);
        else b0[f - 4] = b_read(nxt, 0, f - 4);
      }
      const int idx = x & 15, i = idx >> 2, j = idx & 3;
      if (x < 16)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[i], b0[j], acc[i][j], 0, 0, 0);
      else
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[i], b1[j], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_vmem<0>();  // no load into LDS outlives the loop
  if constexpr (staged_act(ACT)) {
    // Any other activation or a program: through LDS, once every wave is
    // done reading its last stage.
    static_assert(4 * 32 * epi_pitch<WN>() * 4 <= S * STAGE, "staged epilogue fits the stages");
    __syncthreads();
    epilogue_staged<FM, FN, WM, WN, false, ACT == ACT_PROG>(g, (float*)lds, split, batch, m0, n0, wm, wn, wave,
                                                             lane, acc);
  } else {
    epilogue_direct<FM, FN, WM, WN, false, ACT, BF16>(g, split, batch, m0, n0, wm, wn, lane, true, acc);
  }
}

// ---------------------------------------------------------------------------
// 64-wide K stages. The same operand handling with BK = 64 in two LDS stages
// of 64 KiB: every K-contiguous load fetches whole 128-byte pieces of 8 rows,
// so a cache line is requested once even when no other workgroup shares it
// (split-K over long K streams each workgroup's own rows: with 32-wide tiles
// each 64-byte half of a line was a separate request for the same line), and
// a step has one barrier per 64 MFMAs.
// K-contiguous tiles: [256 rows][64 k], 128-byte rows; 16-byte chunk c of row
// r sits in slot c ^ swz64(r), swz64(r) = (r >> 1) & 7, so a fragment read
// (row lane % 32, one chunk) meets distinct banks across 16 lanes. Row-major
// B: [64 k][256 n], 512-byte rows swizzled as in the 32-wide kernel.
//
// NW = 8 waves (the default: two per SIMD, 128 x 64 outputs each) or 4 (one
// per SIMD, 128 x 128). Step t is four k-steps of 16, NS = FM * FN MFMA
// slots each (32 or 64 slots per step). The first FM + FN slots of k-steps
// 0-2 read the next k-step's fragments (two register sets alternate); before
// slot BAR (24 or 44) the wave waits for its loads of stage t + 1 and its
// reads of stage t, and the barrier both publishes stage t + 1 and frees
// stage t; the next LOADS slots issue the loads of stage t + 2 into it and the
// last FM + FN slots read stage t + 1's first fragments. The loads of a stage
// have ~one step to land.
template <int LB, int ACT, bool BF16, int NW, int BN, bool RAGGED = false, int BM = 256, bool TA = false,
          bool NT = false>
__global__ __launch_bounds__(NW * 64, 1) void gemm_bf16_dma64_kernel(GemmArgs g) {
  // B [K, N] row-major, or packed in K-major panels of P columns ([N/P, K, P])
  // or 32 x 32 blocks ([N/32, K/32, 32 k, 32 n]): each lands in LDS as the
  // same row-major [64 k][256 n] tile.
  constexpr bool BPK = LB == L_PANELS || LB == L_BLOCKED;
  constexpr bool BT = LB == L_RCONTIG || BPK;
  constexpr bool VN = LB == L_VNNI_PANELS;         // B in K-pair (VNNI) panels
  constexpr int BK = 64;
  static_assert(BN == 256 || (BN == 128 && NW == 4 && (LB == L_KCONTIG || LB == L_RCONTIG)),
                "256 x 128 and 128 x 128 tiles: four waves, B [N, K] or [K, N]");
  static_assert(BM == 256 || (BM == 128 && BN == 128), "128-row tiles are 128 x 128");
  // TA: A stored [K, M] (op(A) = its transpose): its 64 x 256 stage tiles are
  // loaded and read exactly as row-major B's (512-byte rows, transposing LDS
  // reads), M in place of N.
  static_assert(!TA || (BM == 256 && !RAGGED), "transposed A: whole 256 x 256 tiles");
  static_assert(!RAGGED || LB == L_KCONTIG || LB == L_RCONTIG, "ragged tiles: B [N, K] or [K, N]");
  constexpr int ROWB = BK * 2;                     // bytes per K-contiguous tile row
  constexpr int NROWB = BN * 2;                    // bytes per row-major B tile row
  constexpr int A_BYTES = BM * ROWB;               // 32 KiB (16 KiB for 128-row tiles)
  constexpr int STAGE = A_BYTES + BN * BK * 2;     // 64 KiB (48 or 32 KiB for the smaller tiles)
  // NW = 4: one wave per SIMD, 2 x 2 waves of BM / 2 x BN / 2 outputs; NW = 8:
  // two per SIMD, 2 x 4 waves of 128 x 64.
  constexpr int WM = BM / 2, WN = BN / (NW / 2), FM = WM / 32, FN = WN / 32;
  constexpr int LA = BM / 8 / NW, LBN = BN / 8 / NW;  // 1 KiB loads of A / B per wave per stage
  constexpr int LOADS = LA + LBN;
  constexpr int NS = FM * FN, SLOTS = 4 * NS;      // MFMAs per k-step / per stage
  constexpr int NF = FM + FN;                      // fragment reads per k-step
  // Slot of the stage's wait + barrier: after the last k-step's fragment
  // reads (slot 2 NS + NF), at or before the next stage's first reads (slot
  // SLOTS - NF).
  constexpr int BAR = NS == 16 ? 44 : NS == 8 ? 24 : 12;
  static_assert(BAR >= 2 * NS + NF && BAR <= SLOTS - NF && BAR < SLOTS, "slot plan");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];

  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, g.xcds, tm, tn);
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
  // K-contiguous operands: wave w loads tile rows R w .. R w + R - 1 (R =
  // 256 / NW), 8 rows per load: lane l fills slot l % 8 of row R w + 8 q + l / 8
  // of load q, whose swizzle is (l / 16) | 4 (q & 1). Byte offsets below 2^31:
  // the operands' byte ranges are.
  const int rr = lane >> 3, slot = lane & 7;
  auto kc_voff = [&](int64_t ld, int par) {
    return (int32_t)((rr * ld + (slot ^ ((rr >> 1) | (par << 2))) * 8) * 2);
  };
  int32_t voff_a0, voff_a1, soff_a, blk_a;
  if constexpr (TA) {
    const int r = lane >> 5, c = lane & 31;
    voff_a0 = (int32_t)((r * g.a.ld + (c ^ swz_n(r)) * 8) * 2);      // even q
    voff_a1 = (int32_t)((r * g.a.ld + (c ^ swz_n(r + 2)) * 8) * 2);  // odd q
    soff_a = (int32_t)((wave * (64 / NW) * g.a.ld + m0) * 2);
    blk_a = (int32_t)(2 * g.a.ld * 2);
  } else {
    voff_a0 = kc_voff(g.a.ld, 0);
    voff_a1 = kc_voff(g.a.ld, 1);
    soff_a = (int32_t)((m0 + wave * (BM / NW)) * g.a.ld * 2);
    blk_a = (int32_t)(8 * g.a.ld * 2);
  }
  // RAGGED (M or N not whole tiles): the scalar offset of a buffer load is
  // not range-checked, so rows (columns) past the edge are not addressed at
  // all: each lane's offset holds its whole row (column), clamped to the last
  // row M - 1 (N - 1, or the last 8-column chunk of row-major B), and the
  // scalar offset only the K position. The duplicated rows and columns reach
  // only outputs that are never stored.
  auto kc_voff_clamped = [&](int64_t ld, int64_t row, int64_t rows, int par) {
    return (int32_t)((min(row, rows - 1) * ld + (slot ^ ((rr >> 1) | (par << 2))) * 8) * 2);
  };
  int32_t va[RAGGED ? LA : 1];
  if constexpr (RAGGED) {
#pragma unroll
    for (int q = 0; q < LA; ++q)
      va[q] = kc_voff_clamped(g.a.ld, m0 + wave * (BM / NW) + q * 8 + rr, g.m, q & 1);
  }
  // B: K-contiguous as A; row-major: wave w loads K rows Q w .. Q w + Q - 1
  // (Q = 64 / NW) in pairs Q w + 2 q, Q w + 2 q + 1, lane l filling slot
  // l % 32 of row l / 32 of the pair.
  // VNNI panels of width P ([N/P, Kp/2, P, 2]; the blocked VNNI layout is
  // P = 32): a stage is 32 K pairs x 256 columns. For P <= 256 it is 256 / P
  // runs of 32 pair rows x P columns, each one contiguous 128 P bytes of its
  // panel; for wider panels, 32 pair rows of 256 columns (1 KiB each, 4 P
  // bytes apart). Either way load q of wave w copies 1 KiB, the
  // (LBN w + q)-th of the stage in that order, to LDS unchanged: [256 / PL][32][PL][2] with
  // PL = min(P, 256). Its byte offset is vn_off[q] + (k0 / 2) * 4 P.
  int32_t voff_b0, voff_b1, soff_b, blk_b;
  int32_t vn_off[LBN];
  const int64_t P = g.b.panel;
  const int PL = (int)min<int64_t>(P, 256);
  if constexpr (VN) {
    voff_b0 = voff_b1 = lane * 16;
    soff_b = blk_b = 0;
#pragma unroll
    for (int q = 0; q < LBN; ++q) {
      const int64_t idx = wave * LBN + q;
      int64_t off;
      if (P <= 256) {
        const int64_t b = idx * 1024, run = 128 * P;
        off = ((n0 / P + b / run) * (g.b.kpad / 2)) * 4 * P + b % run;
      } else {
        off = ((n0 / P) * (g.b.kpad / 2) + idx) * 4 * P + (n0 % P) * 4;
      }
      vn_off[q] = (int32_t)off;
    }
  } else if constexpr (BPK) {
    // Element (k, n) sits at col(n) + row(k): col(n) = (n / P) K P + n % P,
    // row(k) = k P (panels); col(n) = (n / 32) (K / 32) 1024 + n % 32,
    // row(k) = (k / 32) 1024 + (k % 32) 32 (blocks). A lane's 8 columns stay
    // in one panel or block (P % 8 == 0), and the two rows of a load (k even,
    // k + 1) are one row stride apart, so the lane offset holds col(n) and the
    // row within the pair, the scalar offset row(k).
    const int r = lane >> 5, c = lane & 31;
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
    // row l / 16; row k % 4 == l / 16 for every load, so one lane offset.
    const int r = lane >> 4, c = lane & 15;
    if constexpr (RAGGED) {
      const int64_t last = ((g.n - 1) >> 3) << 3;  // the last 8-column chunk
      voff_b0 = voff_b1 = (int32_t)((r * g.b.ld + min(n0 + (c ^ swz_n(r)) * 8, last)) * 2);
      soff_b = (int32_t)(wave * (64 / NW) * g.b.ld * 2);
    } else {
      voff_b0 = voff_b1 = (int32_t)((r * g.b.ld + (c ^ swz_n(r)) * 8) * 2);
      soff_b = (int32_t)((wave * (64 / NW) * g.b.ld + n0) * 2);
    }
    blk_b = (int32_t)(4 * g.b.ld * 2);
  } else if constexpr (BT) {
    const int r = lane >> 5, c = lane & 31;
    if constexpr (RAGGED) {
      const int64_t last = ((g.n - 1) >> 3) << 3;  // the last 8-column chunk
      voff_b0 = (int32_t)((r * g.b.ld + min(n0 + (c ^ swz_n(r)) * 8, last)) * 2);
      voff_b1 = (int32_t)((r * g.b.ld + min(n0 + (c ^ swz_n(r + 2)) * 8, last)) * 2);
      soff_b = (int32_t)(wave * (64 / NW) * g.b.ld * 2);
    } else {
      voff_b0 = (int32_t)((r * g.b.ld + (c ^ swz_n(r)) * 8) * 2);      // even q
      voff_b1 = (int32_t)((r * g.b.ld + (c ^ swz_n(r + 2)) * 8) * 2);  // odd q
      soff_b = (int32_t)((wave * (64 / NW) * g.b.ld + n0) * 2);
    }
    blk_b = (int32_t)(2 * g.b.ld * 2);
  } else {
    voff_b0 = kc_voff(g.b.ld, 0);
    voff_b1 = kc_voff(g.b.ld, 1);
    soff_b = (int32_t)((n0 + wave * (BN / NW)) * g.b.ld * 2);
    blk_b = (int32_t)(8 * g.b.ld * 2);
  }
  int32_t vb[RAGGED && !BT && !VN ? LBN : 1];
  if constexpr (RAGGED && !BT && !VN) {
#pragma unroll
    for (int q = 0; q < LBN; ++q)
      vb[q] = kc_voff_clamped(g.b.ld, n0 + wave * (BN / NW) + q * 8 + rr, g.n, q & 1);
  }
  const uint32_t lds_w = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + wave * LA * 1024;
  const uint32_t lds_wb = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + A_BYTES + wave * LBN * 1024;

  // Stage t of the walk is K stage (t + rot) mod ktiles of the chunk.
  const int rot =
      g.k_stagger ? (int)(((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) % (unsigned)ktiles) : 0;
  // DMA q (< LOADS) of stage t: A for q < LA, then B.
  auto dma = [&](int t, int q) {
    int tr = min(t, ktiles - 1) + rot;
    if (tr >= ktiles) tr -= ktiles;
    const int64_t k0 = k_begin + (int64_t)tr * BK;
    const uint32_t st = lds_w + (uint32_t)((t & 1) * STAGE);
    const uint32_t sb = lds_wb + (uint32_t)((t & 1) * STAGE);
    if (q < LA) {
      if constexpr (RAGGED)
        lds_dma16<NT>(srd_a, va[q], (int32_t)(k0 * 2), st + q * 1024);
      else if constexpr (TA)
        lds_dma16<NT>(srd_a, (q & 1) ? voff_a1 : voff_a0, soff_a + q * blk_a + (int32_t)(k0 * g.a.ld * 2),
                  st + q * 1024);
      else
        lds_dma16<NT>(srd_a, (q & 1) ? voff_a1 : voff_a0, soff_a + q * blk_a + (int32_t)(k0 * 2), st + q * 1024);
    } else if constexpr (VN) {
      const int qb = q - LA;
      lds_dma16<NT>(srd_b, voff_b0, vn_off[qb] + (int32_t)((k0 / 2) * 4 * P), sb + qb * 1024);
    } else if constexpr (BPK) {
      const int qb = q - LA;
      const int64_t kr = k0 + wave * (64 / NW) + 2 * qb;  // even
      const int64_t row = LB == L_PANELS ? kr * P : (kr >> 5) * 1024 + (kr & 31) * 32;
      lds_dma16<NT>(srd_b, (qb & 1) ? voff_b1 : voff_b0, (int32_t)(row * 2), sb + qb * 1024);
    } else if constexpr (RAGGED && !BT) {
      const int qb = q - LA;
      lds_dma16<NT>(srd_b, vb[qb], (int32_t)(k0 * 2), sb + qb * 1024);
    } else {
      const int qb = q - LA;
      const int32_t kb = BT ? (int32_t)(k0 * g.b.ld * 2) : (int32_t)(k0 * 2);
      lds_dma16<NT>(srd_b, (qb & 1) ? voff_b1 : voff_b0, soff_b + qb * blk_b + kb,
                sb + qb * 1024);
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment reads. A (and K-contiguous B): row lane % 32 of the fragment,
  // chunk 2 ks + lane / 32 (ks < 4).
  const int frow = lane & 31, fk = lane >> 5, fswz = swz64(frow);
  const uint8_t* a_frag = lds + (wm * WM + frow) * ROWB;
  const uint8_t* b_frag = lds + A_BYTES + (wn * WN + frow) * ROWB;
  int b_tr[FN], a_tr[TA ? FM : 1];
  {
    const int gi = lane >> 4, sl = lane & 15;
    const int v = (2 * (gi & 1) + ((sl & 3) >> 1)) ^ swz_n(sl >> 2);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      b_tr[j] = A_BYTES + (8 * (gi >> 1) + (sl >> 2)) * NROWB + ((wn * (WN / 8) + 4 * j) ^ v) * 16 + 8 * (sl & 1);
    if constexpr (TA) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        a_tr[i] = (8 * (gi >> 1) + (sl >> 2)) * (BM * 2) + ((wm * (WM / 8) + 4 * i) ^ v) * 16 + 8 * (sl & 1);
    }
  }
  // VNNI B: column n = wn * 128 + 32 j + lane % 32 needs K pairs
  // 8 ks + 4 (lane / 32) .. + 3 (4 * PL bytes apart), i.e. K values
  // 16 ks + 8 (lane / 32) .. + 7 -- the MFMA's operand.
  int b_vn[FN];
  const int pair_pitch = 4 * PL;
  if constexpr (VN) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = wn * WN + 32 * j + frow;
      b_vn[j] = A_BYTES + (n / PL) * 32 * pair_pitch + (n % PL) * 4 + 4 * fk * pair_pitch;
    }
  }
  auto a_read = [&](int stage, int ks, int i) -> bf16x8_t {
    if constexpr (TA) {
      const uint8_t* p = lds + stage * STAGE + a_tr[i] + 16 * ks * (BM * 2);
      return __builtin_shufflevector(lds_read_tr(p), lds_read_tr(p + 4 * (BM * 2)), 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      return *(const bf16x8_t*)(a_frag + stage * STAGE + i * 32 * ROWB + ((2 * ks + fk) ^ fswz) * 16);
    }
  };
  auto b_read = [&](int stage, int ks, int j) -> bf16x8_t {
    if constexpr (VN) {
      const uint8_t* p = lds + stage * STAGE + b_vn[j] + 8 * ks * pair_pitch;
      const uint4 v = make_uint4(*(const uint32_t*)p, *(const uint32_t*)(p + pair_pitch),
                                 *(const uint32_t*)(p + 2 * pair_pitch),
                                 *(const uint32_t*)(p + 3 * pair_pitch));
      return __builtin_bit_cast(bf16x8_t, v);
    } else if constexpr (BT) {
      const uint8_t* p = lds + stage * STAGE + b_tr[j] + 16 * ks * NROWB;
      return __builtin_shufflevector(lds_read_tr(p), lds_read_tr(p + 4 * NROWB), 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      return *(const bf16x8_t*)(b_frag + stage * STAGE + j * 32 * ROWB + ((2 * ks + fk) ^ fswz) * 16);
    }
  };

  // The host launches this kernel only with at least one K stage per split.
  bf16x8_t fa[2][FM], fb[2][FN];
#pragma unroll
  for (int q = 0; q < LOADS; ++q) dma(0, q);
#pragma unroll
  for (int q = 0; q < LOADS; ++q) dma(1, q);
  wait_vmem<LOADS>();  // stage 0 landed
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = a_read(0, 0, i);
#pragma unroll
  for (int j = 0; j < FN; ++j) fb[0][j] = b_read(0, 0, j);

  for (int t = 0; t < ktiles; ++t) {
    const int cur = t & 1, nxt = cur ^ 1;
#pragma unroll
    for (int x = 0; x < SLOTS; ++x) {
      __builtin_amdgcn_sched_barrier(0);
      const int ks = x / NS, sub = x % NS;
      if (x == BAR) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (ks < 3 && sub < NF) {
        const int set = (ks + 1) & 1;
        if (sub < FM) fa[set][sub] = a_read(cur, ks + 1, sub);
        else fb[set][sub - FM] = b_read(cur, ks + 1, sub - FM);
      }
      // The stage's loads, spread evenly over the slots after the barrier.
#pragma unroll
      for (int q = (x - BAR) * LOADS / (SLOTS - BAR); q < (x + 1 - BAR) * LOADS / (SLOTS - BAR); ++q)
        if (x >= BAR) dma(t + 2, q);
      if (x >= SLOTS - NF) {
        const int f = x - (SLOTS - NF);
        if (f < FM) fa[0][f] = a_read(nxt, 0, f);
        else fb[0][f - FM] = b_read(nxt, 0, f - FM);
      }
      const int i = sub / FN, j = sub % FN, set = ks & 1;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_vmem<0>();  // no load into LDS outlives the loop
  // RAGGED: tiles that cross M or N store element by element, guarded.
  if constexpr (staged_act(ACT)) {
    // Any other activation or a program: through LDS, once every wave is
    // done reading its last stage.
    static_assert(NW * 32 * epi_pitch<WN>() * 4 <= 2 * STAGE, "staged epilogue fits the stages");
    __syncthreads();
    constexpr bool PROG = ACT == ACT_PROG;
    if (!RAGGED || (m0 + BM <= g.m && n0 + BN <= g.n))
      epilogue_staged<FM, FN, WM, WN, false, PROG>(g, (float*)lds, split, batch, m0, n0, wm, wn, wave, lane, acc);
    else
      epilogue_staged<FM, FN, WM, WN, true, PROG>(g, (float*)lds, split, batch, m0, n0, wm, wn, wave, lane, acc);
  } else {
    if (!RAGGED || (m0 + BM <= g.m && n0 + BN <= g.n))
      epilogue_direct<FM, FN, WM, WN, false, ACT, BF16>(g, split, batch, m0, n0, wm, wn, lane, true, acc);
    else
      epilogue_direct<FM, FN, WM, WN, true, ACT, BF16>(g, split, batch, m0, n0, wm, wn, lane, true, acc);
  }
}

// ---------------------------------------------------------------------------
// The 16x16x32 kernel (body in hmx_gemm_mi16.hpp).
template <int LB, int ACT, bool BF16, bool RAGGED = false, int BM = 256, int BN = 256, int NW = 8, int S = 2>
__global__ __launch_bounds__(NW * 64, 1) void gemm_bf16_mi16_kernel(GemmArgs g) {
  gemm_bf16_mi16_body<LB, ACT, BF16, RAGGED, BM, BN, NW, S>(g);
}

// A product of several rounds of 256 x 256 tiles and a tail of 256 x 128
// tiles in one launch: workgroup b < head_blocks runs head's tile b, the
// others rest's tile b - head_blocks (head_blocks a multiple of the XCD
// count, so the XCD-aware tile order holds for both). Both are multi-round,
// so C is streamed.
template <int LB, int ACT, bool BF16>
__global__ __launch_bounds__(512, 1) void gemm_bf16_mi16_rounds_kernel(GemmArgs head, GemmArgs rest,
                                                                        int head_blocks) {
  constexpr int kHead = mi16_lds_bytes<ACT, 256, 256, 8, 2>(), kTail = mi16_lds_bytes<ACT, 256, 128, 8, 2>();
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kHead > kTail ? kHead : kTail];
  const int b = (int)blockIdx.x;
  if (b < head_blocks)
    gemm_bf16_mi16_body<LB, ACT, BF16, false, 256, 256, 8, 2>(head, lds, b, false);
  else
    gemm_bf16_mi16_body<LB, ACT, BF16, false, 256, 128, 8, 2>(rest, lds, b - head_blocks, false);
}

// ---------------------------------------------------------------------------
// f32 direct-to-LDS kernel (v_mfma_f32_32x32x2_f32) for whole 256 x 256 tiles
// of long-K split-K products: row-major A, B [N, K] or [K, N], f32 partials
// with the identity epilogue. The register-staged f32 kernel has to hold the
// next tile's loads, two waves' fragments and 128 accumulators per wave in
// 256 registers, and the compiler sinks the loads to where they are stored;
// here the loads go straight to LDS, so four waves (one per SIMD, 128 x 128
// outputs each, 256 accumulators in AGPRs) keep two fragment sets in VGPRs.
// With NW = 8 the eight waves (two per SIMD) own 128 x 64 outputs each (128
// accumulators): one wave's MFMAs run while the other of its SIMD waits at
// the stage barrier or on an LDS read.
//
// Stages are 32 K deep (one 128-byte line of each A row), two of 64 KiB:
// K-contiguous tiles [256 rows][32 k] with 16-byte chunk c of row r in slot
// c ^ swz64(r), as the bf16 kernel; row-major B [32 k][256 n], 1 KiB rows with
// chunk c of row k in slot c ^ (8 ((k >> 2) & 1)), so the two half-waves of a
// fragment read (rows k and k + 4, same columns) meet different banks.
//
// A step is K = 8 (four MFMAs of K = 2 for each of the FM x FN fragment
// pairs: 64 slots with four waves, 32 with eight); a stage is four steps. The
// first FM + FN slots of each step read the next step's fragments (two
// register sets alternate). Before step 3 the wave waits for its loads of
// stage t + 1 and its reads of stage t, and the barrier both publishes t + 1
// and frees t; step 3 then reads t + 1's first fragments and issues the
// wave's 16 (8) loads of stage t + 2 into t's buffer from slot 8 on, three
// steps ahead of their use.
template <int LB, int NW = 4, int ACT = ACT_ID, bool BF16 = false>
__global__ __launch_bounds__(NW * 64, 1) void gemm_f32_dma_kernel(GemmArgs g) {
  static_assert(NW == 4 || NW == 8, "f32 waves");
  constexpr bool BT = LB == L_RCONTIG;             // B row-major [K, N]
  constexpr int BM = 256, BN = 256, BK = 32;
  constexpr int ROWB = BK * 4;                     // bytes per K-contiguous tile row
  constexpr int NROWB = BN * 4;                    // bytes per row-major B tile row
  constexpr int A_BYTES = BM * ROWB;               // 32 KiB
  constexpr int STAGE = A_BYTES + BN * BK * 4;     // 64 KiB
  // Four waves of 128 x 128 (2 x 2), or eight of 128 x 64 (2 x 4).
  constexpr int FM = 4, FN = NW == 8 ? 2 : 4, WM = 128, WN = 32 * FN;
  constexpr int LOADS = 64 / NW;                   // DMA instructions per wave per stage
  constexpr int LA = LOADS / 2;                    // of which A
  constexpr int KCR = 256 / NW;                    // K-contiguous tile rows per wave
  constexpr int BTR = 32 / NW;                     // row-major B rows per wave
  constexpr int SLOTS = FM * FN * 4;               // MFMAs per step
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];

  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, g.xcds, tm, tn);
  const int split = blockIdx.y, batch = blockIdx.z;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t k_begin = (int64_t)split * g.k_chunk;
  const int64_t k_end = min(g.k, k_begin + g.k_chunk);
  const int ktiles = (int)((k_end - k_begin) / BK);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / (NW / 2), wn = wave % (NW / 2);

  const i32x4_t srd_a = make_srd((const float*)g.a.p + batch * g.stride_a, g.a.bytes);
  const i32x4_t srd_b = make_srd((const float*)g.b.p + batch * g.stride_b, g.b.bytes);
  // K-contiguous operands: wave w loads tile rows KCR w .. KCR w + KCR - 1,
  // 8 rows of 128 bytes per load (lane l: slot l % 8 of row KCR w + 8 q + l / 8,
  // swizzle (l / 16) | 4 (q & 1)). Byte offsets below 2^31: the operands'
  // byte ranges are.
  const int rr = lane >> 3, slot = lane & 7;
  auto kc_voff = [&](int64_t ld, int par) {
    return (int32_t)((rr * ld + (slot ^ ((rr >> 1) | (par << 2))) * 4) * 4);
  };
  const int32_t voff_a0 = kc_voff(g.a.ld, 0), voff_a1 = kc_voff(g.a.ld, 1);
  const int32_t soff_a = (int32_t)((m0 + wave * KCR) * g.a.ld * 4);
  const int32_t blk_a = (int32_t)(8 * g.a.ld * 4);
  // B: K-contiguous as A; row-major: wave w loads K rows BTR w .. BTR w +
  // BTR - 1, one 1 KiB row per load (lane l: slot l), swizzled by bit 2 of
  // the row.
  int32_t voff_b0, voff_b1, soff_b, blk_b;
  if constexpr (BT) {
    voff_b0 = (int32_t)((n0 + lane * 4) * 4);          // rows with bit 2 clear
    voff_b1 = (int32_t)((n0 + (lane ^ 8) * 4) * 4);    // rows with bit 2 set
    soff_b = (int32_t)(wave * BTR * g.b.ld * 4);
    blk_b = (int32_t)(g.b.ld * 4);
  } else {
    voff_b0 = kc_voff(g.b.ld, 0);
    voff_b1 = kc_voff(g.b.ld, 1);
    soff_b = (int32_t)((n0 + wave * KCR) * g.b.ld * 4);
    blk_b = (int32_t)(8 * g.b.ld * 4);
  }
  const uint32_t lds_w = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + wave * (32 * 1024 / NW);

  // Stage t of the walk is K stage (t + rot) mod ktiles of the chunk.
  const int rot =
      g.k_stagger ? (int)(((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) % (unsigned)ktiles) : 0;
  // DMA q (< LOADS) of stage t: A for q < LA, then B.
  auto dma = [&](int t, int q) {
    int tr = min(t, ktiles - 1) + rot;
    if (tr >= ktiles) tr -= ktiles;
    const int64_t k0 = k_begin + (int64_t)tr * BK;
    const uint32_t st = lds_w + (uint32_t)((t & 1) * STAGE);
    if (q < LA) {
      lds_dma16(srd_a, (q & 1) ? voff_a1 : voff_a0, soff_a + q * blk_a + (int32_t)(k0 * 4), st + q * 1024);
    } else {
      const int qb = q - LA;
      const int32_t kb = BT ? (int32_t)(k0 * g.b.ld * 4) : (int32_t)(k0 * 4);
      const int32_t voff = BT ? ((((BTR * wave + qb) >> 2) & 1) ? voff_b1 : voff_b0)
                              : ((qb & 1) ? voff_b1 : voff_b0);
      lds_dma16(srd_b, voff, soff_b + qb * blk_b + kb, st + A_BYTES + qb * 1024);
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment reads of step k8 (0, 8, 16, 24 within a stage): lane l feeds
  // MFMA s (< 4) the values at K = k8 + 4 (l / 32) + s, row / column l % 32
  // of the fragment.
  const int frow = lane & 31, fk = lane >> 5, fswz = swz64(frow);
  const uint8_t* a_frag = lds + (wm * WM + frow) * ROWB;
  const uint8_t* b_frag = lds + A_BYTES + (wn * WN + frow) * ROWB;
  // Row-major B: column n = wn * 128 + 32 j + l % 32 sits in chunk n / 4 of
  // its row, stored in slot (n / 4) ^ 8 (l / 32) for the rows this lane reads.
  int b_rc[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = wn * WN + 32 * j + frow;
    b_rc[j] = A_BYTES + 4 * fk * NROWB + (((n >> 2) ^ (8 * fk)) << 4) + (n & 3) * 4;
  }
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  auto a_read = [&](int stage, int k8, int i) -> f32x4v {
    return *(const f32x4v*)(a_frag + stage * STAGE + i * 32 * ROWB + (((k8 >> 2) + fk) ^ fswz) * 16);
  };
  auto b_read = [&](int stage, int k8, int j) -> f32x4v {
    if constexpr (BT) {
      const uint8_t* p = lds + stage * STAGE + b_rc[j] + k8 * NROWB;
      return f32x4v{*(const float*)p, *(const float*)(p + NROWB), *(const float*)(p + 2 * NROWB),
                    *(const float*)(p + 3 * NROWB)};
    } else {
      return *(const f32x4v*)(b_frag + stage * STAGE + j * 32 * ROWB + (((k8 >> 2) + fk) ^ fswz) * 16);
    }
  };

  // The host launches this kernel only with at least one K stage per split.
  f32x4v fa[2][FM], fb[2][FN];
#pragma unroll
  for (int q = 0; q < LOADS; ++q) dma(0, q);
#pragma unroll
  for (int q = 0; q < LOADS; ++q) dma(1, q);
  wait_vmem<LOADS>();  // stage 0 landed
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = a_read(0, 0, i);
#pragma unroll
  for (int j = 0; j < FN; ++j) fb[0][j] = b_read(0, 0, j);

  for (int t = 0; t < ktiles; ++t) {
    const int cur = t & 1, nxt = cur ^ 1;
#pragma unroll
    for (int step = 0; step < 4; ++step) {
      const int set = step & 1;
      if (step == 3) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
      for (int x = 0; x < SLOTS; ++x) {
        __builtin_amdgcn_sched_barrier(0);
        if (x < FM + FN) {
          // The next step's fragments: this stage's, or t + 1's first.
          const int stg = step < 3 ? cur : nxt, k8 = step < 3 ? 8 * (step + 1) : 0;
          if (x < FM) fa[set ^ 1][x] = a_read(stg, k8, x);
          else fb[set ^ 1][x - FM] = b_read(stg, k8, x - FM);
        } else if (step == 3 && x >= 8 && x < 8 + LOADS) {
          dma(t + 2, x - 8);
        }
        const int s = x / (FM * FN), idx = x % (FM * FN), i = idx / FN, j = idx % FN;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[set][i][s], fb[set][j][s], acc[i][j], 0, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_vmem<0>();  // no load into LDS outlives the loop
  epilogue_direct<FM, FN, WM, WN, false, ACT, BF16>(g, split, batch, m0, n0, wm, wn, lane, true, acc);
}

// Skinny products: at most 64 rows of row-major A against B [N, K] (a
// decode-shaped linear layer, batch 1), bound by reading B once. A workgroup
// owns 32 RB rows of B (32 RB columns of C); its NW waves split K into NW ranges
// of whole 64-element stages and each streams its own range with no
// workgroup barrier: D stages in flight, D + 1 ring slots of LDS per wave
// (D = 1 or 2: deeper queues measured slower).
// A slot holds the B tile [32 RB n][64 k] (4 RB KiB) and A rows [8 XL][64 k]: the
// rows of A the product has (XL = 1, 2, 4 or 8 loads of 8 rows; rows past M
// repeat row M - 1, fragment rows past 8 XL repeat the first 8 XL), in the
// same 128-byte swizzled rows as the GEMM tiles (chunk c of row r in slot
// c ^ swz64(r)), so every load fetches whole 128-byte pieces of 8 rows.
//
// Each stage is four v_mfma_f32_32x32x16_bf16 per pair of 32-row blocks of B
// (rb) and A (mb; two blocks past 32 rows) with B's rows as the first
// operand, giving C transposed: element e of lane l of tile (rb, mb) is
// column n0 + 32 rb + 8 (e / 4) + 4 (l / 32) + e % 4 of C row 32 mb + l % 32.
// After the loop the waves' accumulators meet in LDS and are summed in wave
// order (so results do not depend on timing); the groups of four elements
// e / 4 of every tile are dealt to the waves in turn, each finishing its
// groups (bias, scale, shift, the activation, one rounding) and storing four
// adjacent columns at a time.
template <int NW, int XL, int D, int RB>
__global__ __launch_bounds__(NW * 64) void gemm_bf16_skinny_kernel(GemmArgs g) {
  static_assert((NW == 2 || NW == 4) && (XL == 1 || XL == 2 || XL == 4 || XL == 8) && (RB == 1 || RB == 2),
                "skinny shape");
  constexpr int MB = XL == 8 ? 2 : 1;          // 32-row blocks of A (columns of the MFMA)
  constexpr int BB = 4096 * RB;                // bytes of B per stage: [32 RB n][64 k]
  constexpr int L = 4 * RB + XL;               // loads per stage per wave
  constexpr int SB = BB + 1024 * XL;           // bytes per ring slot
  constexpr int RING = (D + 1) * SB;           // bytes per wave
  static_assert(L * D < 64 && NW * RING <= 160 * 1024 && RB * MB * 64 * 64 <= RING, "skinny LDS plan");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NW * RING];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n0 = (int64_t)blockIdx.x * (32 * RB);
  const int stages = (int)(g.k / 64);
  const int t0 = wave * stages / NW, count = (wave + 1) * stages / NW - t0;

  const i32x4_t srd_a = make_srd(g.a.p, g.a.bytes);
  const i32x4_t srd_b = make_srd(g.b.p, g.b.bytes);
  // Load q of a stage fills 8 rows: lane l slot l % 8 of row 8 q + l / 8,
  // clamped to the operand's last row. The lane offset holds the row; the
  // scalar offset (not range-checked) only the stage's K position.
  const int rr = lane >> 3, slot = lane & 7;
  int32_t voff_b[4 * RB], voff_a[XL];
#pragma unroll
  for (int q = 0; q < 4 * RB; ++q) {
    const int r = 8 * q + rr;
    voff_b[q] = (int32_t)((min(n0 + r, g.n - 1) * g.b.ld + (slot ^ swz64(r)) * 8) * 2);
  }
#pragma unroll
  for (int q = 0; q < XL; ++q) {
    const int r = 8 * q + rr;
    voff_a[q] = (int32_t)((min((int64_t)r, g.m - 1) * g.a.ld + (slot ^ swz64(r)) * 8) * 2);
  }
  const uint32_t ring = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + wave * RING;
  // Workgroup b walks its waves' ranges from stage b mod count on, wrapping
  // around: the workgroups in flight then read different K positions of
  // their rows instead of one 128-byte column of B at a time.
  const int rot = (int)(blockIdx.x % (unsigned)max(count, 1));
  auto issue = [&](int u) {
    int uu = u + rot;
    if (uu >= count) uu -= count;
    const int32_t kb = (t0 + uu) * 128;
    const uint32_t st = ring + (uint32_t)((u % (D + 1)) * SB);
#pragma unroll
    for (int q = 0; q < 4 * RB; ++q) lds_dma16(srd_b, voff_b[q], kb, st + q * 1024);
#pragma unroll
    for (int q = 0; q < XL; ++q) lds_dma16(srd_a, voff_a[q], kb, st + BB + q * 1024);
  };

  // Fragment reads of MFMA s: row l % 32, chunk 2 s + l / 32 (K 16 s + 8 (l / 32) ..).
  // (Rows 32 rb + l % 32 of B share the swizzle of row l % 32.)
  const int fr = lane & 31, fh = lane >> 5;
  const int b_off = fr * 128, b_swz = swz64(fr);
  int a_off[MB], a_swz[MB];
  f32x16_t acc[RB][MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int ar = MB == 2 ? 32 * mb + fr : fr & (8 * XL - 1);
    a_off[mb] = BB + ar * 128;
    a_swz[mb] = swz64(ar);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[rb][mb][e] = 0.f;
  }
  if (count > 0) {
#pragma unroll
    for (int u = 0; u < D; ++u)
      if (u < count) issue(u);
    for (int u = 0; u < count; ++u) {
      if (u + D < count) {
        issue(u + D);  // into the slot read in step u - 1
        wait_vmem<L * D>();
      } else {
        wait_vmem<0>();
      }
      const uint8_t* st = lds + wave * RING + (u % (D + 1)) * SB;
      bf16x8_t fb[RB][4], fa[MB][4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          fb[rb][s] = *(const bf16x8_t*)(st + rb * 4096 + b_off + (((2 * s + fh) ^ b_swz) << 4));
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          fa[mb][s] = *(const bf16x8_t*)(st + a_off[mb] + (((2 * s + fh) ^ a_swz[mb]) << 4));
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[rb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[rb][s], fa[mb][s], acc[rb][mb], 0, 0, 0);
    }
  }

  // Every wave's loads have landed (wait_vmem<0> ends its loop) and its ring
  // reads have been consumed; the ring becomes the reduction buffer.
  __syncthreads();
  // Tile t = RB * MB + ... of wave w at red[((w * RB * MB + t) * 16 + e) * 64 + lane].
  constexpr int TILES = RB * MB;
  float* red = (float*)lds;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[((wave * TILES + rb * MB + mb) * 16 + e) * 64 + lane] = acc[rb][mb][e];
  __syncthreads();
  // Unit u (< 4 TILES: group u % 4 of tile u / 4) goes to wave u % NW.
#pragma unroll
  for (int j = 0; j < 4 * TILES / NW; ++j) {
    const int u = wave + NW * j, t = u >> 2, grp = u & 3;
    const int rb = t / MB, mb = t % MB;
    const int64_t row = 32 * mb + fr;
    if (row >= g.m) continue;
    const int64_t col0 = n0 + 32 * rb + 8 * grp + 4 * fh;
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int e = 4 * grp + c;
      float sum = red[(t * 16 + e) * 64 + lane];
#pragma unroll
      for (int w = 1; w < NW; ++w) sum += red[((w * TILES + t) * 16 + e) * 64 + lane];
      float bias, scale, shift;
      column_vectors(g, col0 + c, col0 + c < g.n, bias, scale, shift);
      v[c] = apply_activation(g.act, (sum + bias) * scale + shift, g.act_arg);
    }
    if (g.c_dtype == HMX_DTYPE_BF16) {
      uint16_t* p = (uint16_t*)g.c + row * g.ldc + col0;
      if (col0 + 3 < g.n && (((uintptr_t)p) & 7) == 0) {
        *(uint2*)p = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (col0 + c < g.n) p[c] = (uint16_t)f32_to_bf16_bits(v[c]);
      }
    } else {
      float* p = (float*)g.c + row * g.ldc + col0;
      if (col0 + 3 < g.n && (((uintptr_t)p) & 15) == 0) {
        *(float4*)p = float4{v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (col0 + c < g.n) p[c] = v[c];
      }
    }
  }
}

// The 16x16x32 MFMA kernel for the eight-wave 256 x 256 tiles unless the
// environment sets HMX_GEMM_MFMA=32 (the 32x32x16 kernel, for comparison).
bool mfma16_enabled() {
  static const bool on = [] {
    const char* e = getenv("HMX_GEMM_MFMA");
    return !(e && e[0] == '3');
  }();
  return on;
}

// The 16x16x32 kernel's conditions beyond its template's: no stagger, and
// bf16 C in 16-byte row pieces.
bool mi16_args_ok(const GemmArgs& g) {
  const bool rows16 = g.c_dtype != HMX_DTYPE_BF16 || ((((uintptr_t)g.c) & 15) == 0 && g.ldc % 8 == 0 &&
                                                      g.stride_c % 8 == 0 && g.stride_split % 8 == 0);
  return !g.k_stagger && rows16 && mfma16_enabled();
}

// Eight waves (two per SIMD) unless the environment sets HMX_GEMM_WAVES=4:
// the second wave of a SIMD issues MFMAs while the first waits at the stage
// barrier or on an LDS read (measured: 2-5 % faster on configs 3-5).
bool eight_waves() {
  static const bool eight = [] {
    const char* e = getenv("HMX_GEMM_WAVES");
    return !(e && e[0] == '4');
  }();
  return eight;
}

template <int LB, bool BF16, bool K64, int NW = 4>
void launch_bf16_dma_c(const GemmArgs& g, dim3 grid, hipStream_t s) {
  if constexpr (K64 && NW == 8 &&
                (LB == L_KCONTIG || LB == L_RCONTIG || LB == L_VNNI_PANELS || LB == L_PANELS || LB == L_BLOCKED)) {
    if (mi16_args_ok(g)) {
      switch (g.act) {
        case HMX_EPI_IDENTITY: launch(gemm_bf16_mi16_kernel<LB, ACT_ID, BF16>, grid, 512, s, g); return;
        case HMX_EPI_RELU: launch(gemm_bf16_mi16_kernel<LB, ACT_RELU, BF16>, grid, 512, s, g); return;
        case HMX_EPI_SILU: launch(gemm_bf16_mi16_kernel<LB, ACT_SILU, BF16>, grid, 512, s, g); return;
        default:
          // Other epilogues: compiled into the register epilogue at run
          // time; else the staged epilogue, which stores 16-byte runs of C
          // rows (f32 C: 4-element aligned rows too).
          if (launch_mi16_jit(g, LB, BF16, false, 256, 256, 8, 2, grid, s) == HMX_OK) return;
          if (BF16 || ((((uintptr_t)g.c) & 15) == 0 && g.ldc % 4 == 0 && g.stride_c % 4 == 0 &&
                       g.stride_split % 4 == 0)) {
            if (g.act == HMX_EPI_PROGRAM) launch(gemm_bf16_mi16_kernel<LB, ACT_PROG, BF16>, grid, 512, s, g);
            else launch(gemm_bf16_mi16_kernel<LB, ACT_ANY, BF16>, grid, 512, s, g);
            return;
          }
          break;
      }
    }
  }
  if constexpr (K64) {
    if constexpr (!BF16 && NW == 8 && (LB == L_KCONTIG || LB == L_RCONTIG)) {
      // Split-K grids of one tile per slice (k_stagger): no other workgroup
      // reads a workgroup's operand rows, so its loads are non-temporal.
      if (g.k_stagger && g.act == HMX_EPI_IDENTITY) {
        launch(gemm_bf16_dma64_kernel<LB, ACT_ID, false, 8, 256, false, 256, false, true>, grid, NW * 64, s, g);
        return;
      }
    }
    switch (g.act) {
      case HMX_EPI_RELU: launch(gemm_bf16_dma64_kernel<LB, ACT_RELU, BF16, NW, 256>, grid, NW * 64, s, g); break;
      case HMX_EPI_SILU: launch(gemm_bf16_dma64_kernel<LB, ACT_SILU, BF16, NW, 256>, grid, NW * 64, s, g); break;
      case HMX_EPI_IDENTITY: launch(gemm_bf16_dma64_kernel<LB, ACT_ID, BF16, NW, 256>, grid, NW * 64, s, g); break;
      default:
        if (g.act == HMX_EPI_PROGRAM) launch(gemm_bf16_dma64_kernel<LB, ACT_PROG, BF16, NW, 256>, grid, NW * 64, s, g);
        else launch(gemm_bf16_dma64_kernel<LB, ACT_ANY, BF16, NW, 256>, grid, NW * 64, s, g);
        break;
    }
  } else if constexpr (LB != L_VNNI_PANELS) {
    switch (g.act) {
      case HMX_EPI_RELU: launch(gemm_bf16_dma_kernel<LB, ACT_RELU, BF16>, grid, 256, s, g); break;
      case HMX_EPI_SILU: launch(gemm_bf16_dma_kernel<LB, ACT_SILU, BF16>, grid, 256, s, g); break;
      case HMX_EPI_IDENTITY: launch(gemm_bf16_dma_kernel<LB, ACT_ID, BF16>, grid, 256, s, g); break;
      default:
        if (g.act == HMX_EPI_PROGRAM) launch(gemm_bf16_dma_kernel<LB, ACT_PROG, BF16>, grid, 256, s, g);
        else launch(gemm_bf16_dma_kernel<LB, ACT_ANY, BF16>, grid, 256, s, g);
        break;
    }
  }
}

template <int LB, bool K64>
void launch_bf16_dma_b(const GemmArgs& g, dim3 grid, hipStream_t s) {
  if (eight_waves() && K64) {
    if (g.c_dtype == HMX_DTYPE_BF16)
      launch_bf16_dma_c<LB, true, K64, 8>(g, grid, s);
    else
      launch_bf16_dma_c<LB, false, K64, 8>(g, grid, s);
    return;
  }
  if (g.c_dtype == HMX_DTYPE_BF16)
    launch_bf16_dma_c<LB, true, K64>(g, grid, s);
  else
    launch_bf16_dma_c<LB, false, K64>(g, grid, s);
}

// The 64-wide kernel takes every K chunk of whole 64-element stages unless the
// environment sets HMX_GEMM_DMA64=0 (which keeps the 32-wide kernel, for
// comparison).
bool dma64_enabled() {
  static const bool on = [] {
    const char* e = getenv("HMX_GEMM_DMA64");
    return !(e && e[0] == '0');
  }();
  return on;
}

}  // namespace

bool gemm_bf16_dma_packed_ok(const GemmArgs& g, int lb) {
  if (!(g.k_chunk % 64 == 0 && g.k % 64 == 0 && dma64_enabled())) return false;
  if (lb == L_PANELS) return g.b.panel % 8 == 0;
  if (lb == L_BLOCKED) return true;
  if (lb != L_VNNI_PANELS && lb != L_BLOCKED_VNNI) return false;
  const int64_t p = lb == L_BLOCKED_VNNI ? 32 : g.b.panel;
  return g.b.kpad % 2 == 0 && p % 32 == 0 && (256 % p == 0 || p % 256 == 0);
}

template <int LB, bool BF16>
void launch_bf16_dma_narrow(const GemmArgs& g, dim3 grid, hipStream_t s) {
  // Eight waves of 128 x 32 (two per SIMD): config 4's tail 60.5 -> 58.8 us
  // against four of 128 x 64.
  if (mi16_args_ok(g)) {
    switch (g.act) {
      case HMX_EPI_IDENTITY:
        launch(gemm_bf16_mi16_kernel<LB, ACT_ID, BF16, false, 256, 128, 8>, grid, 512, s, g);
        return;
      case HMX_EPI_RELU:
        launch(gemm_bf16_mi16_kernel<LB, ACT_RELU, BF16, false, 256, 128, 8>, grid, 512, s, g);
        return;
      case HMX_EPI_SILU:
        launch(gemm_bf16_mi16_kernel<LB, ACT_SILU, BF16, false, 256, 128, 8>, grid, 512, s, g);
        return;
      default:
        if (launch_mi16_jit(g, LB, BF16, false, 256, 128, 8, 2, grid, s) == HMX_OK) return;
        break;
    }
  }
  switch (g.act) {
    case HMX_EPI_RELU: launch(gemm_bf16_dma64_kernel<LB, ACT_RELU, BF16, 4, 128>, grid, 256, s, g); break;
    case HMX_EPI_SILU: launch(gemm_bf16_dma64_kernel<LB, ACT_SILU, BF16, 4, 128>, grid, 256, s, g); break;
    case HMX_EPI_IDENTITY: launch(gemm_bf16_dma64_kernel<LB, ACT_ID, BF16, 4, 128>, grid, 256, s, g); break;
    default:
        if (g.act == HMX_EPI_PROGRAM) launch(gemm_bf16_dma64_kernel<LB, ACT_PROG, BF16, 4, 128>, grid, 256, s, g);
        else launch(gemm_bf16_dma64_kernel<LB, ACT_ANY, BF16, 4, 128>, grid, 256, s, g);
        break;
  }
}

// One launch for the whole rounds and the tail unless the environment sets
// HMX_GEMM_FUSED_ROUNDS=0 (two launches, for comparison).
static bool fused_rounds_enabled() {
  static const bool on = [] {
    const char* e = getenv("HMX_GEMM_FUSED_ROUNDS");
    return !(e && e[0] == '0');
  }();
  return on;
}

bool launch_gemm_bf16_dma_rounds(const GemmArgs& head, const GemmArgs& rest, int lb, unsigned head_blocks,
                                 unsigned rest_blocks, hipStream_t s) {
  // The conditions under which launch_gemm_bf16_dma and _narrow both take the
  // 16x16x32 kernel (its prebuilt named activations, or any other epilogue
  // compiled in at run time).
  const bool k64 = head.k_chunk % 64 == 0 && head.k % 64 == 0 && dma64_enabled();
  const bool named = head.act == HMX_EPI_IDENTITY || head.act == HMX_EPI_RELU || head.act == HMX_EPI_SILU;
  if (!fused_rounds_enabled() || !k64 || !eight_waves() || !mi16_args_ok(head) || !mi16_args_ok(rest) ||
      (lb != L_KCONTIG && lb != L_RCONTIG) || head_blocks % (unsigned)std::max(head.xcds, 1) != 0 ||
      head.m % 256 != 0 || head.n % 256 != 0)
    return false;
  // Other epilogues (programs, the other activations): the same launch with
  // the epilogue compiled in, where run-time compilation is on.
  if (!named)
    return launch_mi16_rounds_jit(head, rest, lb, head.c_dtype == HMX_DTYPE_BF16, head_blocks, rest_blocks, s) ==
           HMX_OK;
  const dim3 grid(head_blocks + rest_blocks);
  const int hb = (int)head_blocks;
  auto go = [&](auto lb_c, auto bf16_c) {
    constexpr int LBc = decltype(lb_c)::value;
    constexpr bool BF = decltype(bf16_c)::value;
    switch (head.act) {
      case HMX_EPI_RELU: launch(gemm_bf16_mi16_rounds_kernel<LBc, ACT_RELU, BF>, grid, 512, s, head, rest, hb); break;
      case HMX_EPI_SILU: launch(gemm_bf16_mi16_rounds_kernel<LBc, ACT_SILU, BF>, grid, 512, s, head, rest, hb); break;
      default: launch(gemm_bf16_mi16_rounds_kernel<LBc, ACT_ID, BF>, grid, 512, s, head, rest, hb); break;
    }
  };
  const bool bf16 = head.c_dtype == HMX_DTYPE_BF16;
  if (lb == L_RCONTIG) {
    if (bf16) go(std::integral_constant<int, L_RCONTIG>{}, std::true_type{});
    else go(std::integral_constant<int, L_RCONTIG>{}, std::false_type{});
  } else {
    if (bf16) go(std::integral_constant<int, L_KCONTIG>{}, std::true_type{});
    else go(std::integral_constant<int, L_KCONTIG>{}, std::false_type{});
  }
  return true;
}

void launch_gemm_bf16_dma_narrow(const GemmArgs& g, int lb, dim3 grid, hipStream_t s) {
  const bool bf16 = g.c_dtype == HMX_DTYPE_BF16;
  if (lb == L_RCONTIG) {
    if (bf16) launch_bf16_dma_narrow<L_RCONTIG, true>(g, grid, s);
    else launch_bf16_dma_narrow<L_RCONTIG, false>(g, grid, s);
  } else {
    if (bf16) launch_bf16_dma_narrow<L_KCONTIG, true>(g, grid, s);
    else launch_bf16_dma_narrow<L_KCONTIG, false>(g, grid, s);
  }
}

// Output not a whole number of 256 x 256 tiles (K chunks of whole 64-element
// stages, B K-contiguous or row-major): the eight-wave kernel with clamped
// edge rows and columns and the guarded edge epilogue.
template <int LB, bool BF16>
void launch_bf16_dma_ragged(const GemmArgs& g, dim3 grid, hipStream_t s) {
  if (eight_waves() && mi16_args_ok(g)) {
    switch (g.act) {
      case HMX_EPI_IDENTITY: launch(gemm_bf16_mi16_kernel<LB, ACT_ID, BF16, true>, grid, 512, s, g); return;
      case HMX_EPI_RELU: launch(gemm_bf16_mi16_kernel<LB, ACT_RELU, BF16, true>, grid, 512, s, g); return;
      case HMX_EPI_SILU: launch(gemm_bf16_mi16_kernel<LB, ACT_SILU, BF16, true>, grid, 512, s, g); return;
      default:
        if (launch_mi16_jit(g, LB, BF16, true, 256, 256, 8, 2, grid, s) == HMX_OK) return;
        break;
    }
  }
  switch (g.act) {
    case HMX_EPI_RELU: launch(gemm_bf16_dma64_kernel<LB, ACT_RELU, BF16, 8, 256, true>, grid, 512, s, g); break;
    case HMX_EPI_SILU: launch(gemm_bf16_dma64_kernel<LB, ACT_SILU, BF16, 8, 256, true>, grid, 512, s, g); break;
    case HMX_EPI_IDENTITY: launch(gemm_bf16_dma64_kernel<LB, ACT_ID, BF16, 8, 256, true>, grid, 512, s, g); break;
    default:
        if (g.act == HMX_EPI_PROGRAM) launch(gemm_bf16_dma64_kernel<LB, ACT_PROG, BF16, 8, 256, true>, grid, 512, s, g);
        else launch(gemm_bf16_dma64_kernel<LB, ACT_ANY, BF16, 8, 256, true>, grid, 512, s, g);
        break;
  }
}

// 128 x 128 tiles (four waves of 64 x 64), B K-contiguous or row-major, whole
// or ragged.
// Stages in LDS of the 16x16x32 kernel's 128 x 128 tiles: 4 (one workgroup
// per CU, three stages in flight) or 2 (two workgroups per CU);
// HMX_MI16_STAGES=2 or 4 overrides the choice, for comparison.
int mi16_stages128(const GemmArgs& g, dim3 grid) {
  static const int forced = [] {
    const char* e = getenv("HMX_MI16_STAGES");
    return e ? atoi(e) : 0;
  }();
  if (forced == 2 || forced == 4) return forced;
  return (int64_t)grid.x * grid.y * grid.z <= g.cus ? 4 : 2;
}

template <int LB, bool BF16, bool RAGGED, int S>
bool launch_mi16_128(const GemmArgs& g, dim3 grid, hipStream_t s) {
  switch (g.act) {
    case HMX_EPI_IDENTITY: launch(gemm_bf16_mi16_kernel<LB, ACT_ID, BF16, RAGGED, 128, 128, 4, S>, grid, 256, s, g); return true;
    case HMX_EPI_RELU: launch(gemm_bf16_mi16_kernel<LB, ACT_RELU, BF16, RAGGED, 128, 128, 4, S>, grid, 256, s, g); return true;
    case HMX_EPI_SILU: launch(gemm_bf16_mi16_kernel<LB, ACT_SILU, BF16, RAGGED, 128, 128, 4, S>, grid, 256, s, g); return true;
    default: return false;
  }
}

template <int LB, bool BF16, bool RAGGED>
void launch_bf16_dma128_c(const GemmArgs& g, dim3 grid, hipStream_t s) {
  // The 16x16x32 kernel from 16 stages per split on (1000 x 4096 x 4096:
  // 51 -> 44 us); short chunks (1024^3 split four ways: 16 -> 17.5 us) keep
  // the 32x32x16 kernel.
  if (mi16_args_ok(g) && g.k_chunk >= 16 * 64) {
    const int stages = mi16_stages128(g, grid);
    const bool done = stages == 4 ? launch_mi16_128<LB, BF16, RAGGED, 4>(g, grid, s)
                                  : launch_mi16_128<LB, BF16, RAGGED, 2>(g, grid, s);
    if (done || launch_mi16_jit(g, LB, BF16, RAGGED, 128, 128, 4, stages, grid, s) == HMX_OK) return;
  }
  switch (g.act) {
    case HMX_EPI_RELU: launch(gemm_bf16_dma64_kernel<LB, ACT_RELU, BF16, 4, 128, RAGGED, 128>, grid, 256, s, g); break;
    case HMX_EPI_SILU: launch(gemm_bf16_dma64_kernel<LB, ACT_SILU, BF16, 4, 128, RAGGED, 128>, grid, 256, s, g); break;
    case HMX_EPI_IDENTITY: launch(gemm_bf16_dma64_kernel<LB, ACT_ID, BF16, 4, 128, RAGGED, 128>, grid, 256, s, g); break;
    default:
        if (g.act == HMX_EPI_PROGRAM) launch(gemm_bf16_dma64_kernel<LB, ACT_PROG, BF16, 4, 128, RAGGED, 128>, grid, 256, s, g);
        else launch(gemm_bf16_dma64_kernel<LB, ACT_ANY, BF16, 4, 128, RAGGED, 128>, grid, 256, s, g);
        break;
  }
}

template <int LB>
void launch_bf16_dma128_b(const GemmArgs& g, dim3 grid, hipStream_t s) {
  const bool ragged = g.m % 128 != 0 || g.n % 128 != 0;
  const bool bf16 = g.c_dtype == HMX_DTYPE_BF16;
  if (ragged) {
    if (bf16) launch_bf16_dma128_c<LB, true, true>(g, grid, s);
    else launch_bf16_dma128_c<LB, false, true>(g, grid, s);
  } else {
    if (bf16) launch_bf16_dma128_c<LB, true, false>(g, grid, s);
    else launch_bf16_dma128_c<LB, false, false>(g, grid, s);
  }
}

void launch_gemm_bf16_dma128(const GemmArgs& g, int lb, dim3 grid, hipStream_t s) {
  if (lb == L_RCONTIG)
    launch_bf16_dma128_b<L_RCONTIG>(g, grid, s);
  else
    launch_bf16_dma128_b<L_KCONTIG>(g, grid, s);
}

// A stored [K, M] (trans_a), whole 256 x 256 tiles, K chunks of whole
// 64-element stages, B K-contiguous or row-major: eight waves.
template <int LB, bool BF16>
void launch_bf16_dma_ta_c(const GemmArgs& g, dim3 grid, hipStream_t s) {
  switch (g.act) {
    case HMX_EPI_RELU: launch(gemm_bf16_dma64_kernel<LB, ACT_RELU, BF16, 8, 256, false, 256, true>, grid, 512, s, g); break;
    case HMX_EPI_SILU: launch(gemm_bf16_dma64_kernel<LB, ACT_SILU, BF16, 8, 256, false, 256, true>, grid, 512, s, g); break;
    case HMX_EPI_IDENTITY: launch(gemm_bf16_dma64_kernel<LB, ACT_ID, BF16, 8, 256, false, 256, true>, grid, 512, s, g); break;
    default:
        if (g.act == HMX_EPI_PROGRAM) launch(gemm_bf16_dma64_kernel<LB, ACT_PROG, BF16, 8, 256, false, 256, true>, grid, 512, s, g);
        else launch(gemm_bf16_dma64_kernel<LB, ACT_ANY, BF16, 8, 256, false, 256, true>, grid, 512, s, g);
        break;
  }
}

void launch_gemm_bf16_dma_ta(const GemmArgs& g, int lb, dim3 grid, hipStream_t s) {
  const bool bf16 = g.c_dtype == HMX_DTYPE_BF16;
  if (lb == L_RCONTIG) {
    if (bf16) launch_bf16_dma_ta_c<L_RCONTIG, true>(g, grid, s);
    else launch_bf16_dma_ta_c<L_RCONTIG, false>(g, grid, s);
  } else {
    if (bf16) launch_bf16_dma_ta_c<L_KCONTIG, true>(g, grid, s);
    else launch_bf16_dma_ta_c<L_KCONTIG, false>(g, grid, s);
  }
}

void launch_gemm_bf16_dma(const GemmArgs& g, int lb, dim3 grid, hipStream_t s) {
  if (g.m % 256 != 0 || g.n % 256 != 0) {
    const bool bf16 = g.c_dtype == HMX_DTYPE_BF16;
    if (lb == L_RCONTIG) {
      if (bf16) launch_bf16_dma_ragged<L_RCONTIG, true>(g, grid, s);
      else launch_bf16_dma_ragged<L_RCONTIG, false>(g, grid, s);
    } else {
      if (bf16) launch_bf16_dma_ragged<L_KCONTIG, true>(g, grid, s);
      else launch_bf16_dma_ragged<L_KCONTIG, false>(g, grid, s);
    }
    return;
  }
  if (lb == L_VNNI_PANELS || lb == L_BLOCKED_VNNI) {
    // The blocked VNNI layout [N/32, Kp/32, 16, 32, 2] is VNNI panels of 32.
    GemmArgs v = g;
    if (lb == L_BLOCKED_VNNI) v.b.panel = 32;
    launch_bf16_dma_b<L_VNNI_PANELS, true>(v, grid, s);
    return;
  }
  if (lb == L_PANELS) {
    launch_bf16_dma_b<L_PANELS, true>(g, grid, s);
    return;
  }
  if (lb == L_BLOCKED) {
    launch_bf16_dma_b<L_BLOCKED, true>(g, grid, s);
    return;
  }
  const bool k64 = g.k_chunk % 64 == 0 && g.k % 64 == 0 && dma64_enabled();
  if (lb == L_RCONTIG) {
    if (k64) launch_bf16_dma_b<L_RCONTIG, true>(g, grid, s);
    else launch_bf16_dma_b<L_RCONTIG, false>(g, grid, s);
  } else {
    if (k64) launch_bf16_dma_b<L_KCONTIG, true>(g, grid, s);
    else launch_bf16_dma_b<L_KCONTIG, false>(g, grid, s);
  }
}

template <int NW, int D, int RB>
void launch_bf16_skinny(const GemmArgs& g, hipStream_t s) {
  const dim3 grid((unsigned)ceil_div(g.n, 32 * RB));
  if (g.m <= 8)
    launch(gemm_bf16_skinny_kernel<NW, 1, D, RB>, grid, NW * 64, s, g);
  else if (g.m <= 16)
    launch(gemm_bf16_skinny_kernel<NW, 2, D, RB>, grid, NW * 64, s, g);
  else if (g.m <= 32)
    launch(gemm_bf16_skinny_kernel<NW, 4, D, RB>, grid, NW * 64, s, g);
  else
    launch(gemm_bf16_skinny_kernel<NW, 8, D, RB>, grid, NW * 64, s, g);
}

// Up to one group of 32 B rows per CU (256 on MI355X): four waves
// of 32 rows, two stages in flight each; more: four waves of 64 rows (two
// 32-row blocks share each A fragment, halving A's share of the loads), one
// stage in flight. Measured with graph replay on one box, M x N x K (torch /
// hipBLASLt in brackets): 32 x 4096 x 4096 8.6 us (9.6), 64 x 4096 x 4096
// 12.0 us (11.9); 32 x 11008 x 4096 16.7 us (17.8), 64 x 11008 x 4096 19.9 us
// (19.4), 32 x 28672 x 8192 85.0 us (131.6), 64 x 28672 x 8192 99.4 us
// (99.1). Alternatives on the large shapes: two waves of 32 rows with one
// stage 16.9 / 22.4 / 92.2 / 126.3 us, four waves of 32 rows 18.0 / 24.2 /
// 95.9 / 119.9 us; two stages in flight or more measured slower there.
void launch_gemm_bf16_skinny(const GemmArgs& g, hipStream_t s) {
  if (ceil_div(g.n, 32) <= g.cus)
    launch_bf16_skinny<4, 2, 1>(g, s);
  else
    launch_bf16_skinny<4, 1, 2>(g, s);
}

void launch_gemm_f32_dma(const GemmArgs& g, int lb, dim3 grid, hipStream_t s) {
  // Eight waves (two per SIMD) unless the environment sets HMX_F32_WAVES=4:
  // config 5 (bmm [16, 256, 65536] x [16, 65536, 256]) 0.987 -> 0.970 ms.
  static const int waves = [] {
    const char* e = getenv("HMX_F32_WAVES");
    return e && e[0] == '4' ? 4 : 8;
  }();
  if (waves == 8) {
    // Unsplit products finish C in the kernel (f32 or bf16, a register
    // activation); split-K partials are f32 with the identity epilogue.
    auto go = [&](auto lb_c) {
      constexpr int LBc = decltype(lb_c)::value;
      const bool bf16 = g.c_dtype == HMX_DTYPE_BF16;
      switch (g.act) {
        case HMX_EPI_RELU:
          if (bf16) launch(gemm_f32_dma_kernel<LBc, 8, ACT_RELU, true>, grid, 512, s, g);
          else launch(gemm_f32_dma_kernel<LBc, 8, ACT_RELU, false>, grid, 512, s, g);
          break;
        case HMX_EPI_SILU:
          if (bf16) launch(gemm_f32_dma_kernel<LBc, 8, ACT_SILU, true>, grid, 512, s, g);
          else launch(gemm_f32_dma_kernel<LBc, 8, ACT_SILU, false>, grid, 512, s, g);
          break;
        default:
          if (bf16) launch(gemm_f32_dma_kernel<LBc, 8, ACT_ID, true>, grid, 512, s, g);
          else launch(gemm_f32_dma_kernel<LBc, 8, ACT_ID, false>, grid, 512, s, g);
          break;
      }
    };
    if (lb == L_RCONTIG) go(std::integral_constant<int, L_RCONTIG>{});
    else go(std::integral_constant<int, L_KCONTIG>{});
    return;
  }
  if (lb == L_RCONTIG)
    launch(gemm_f32_dma_kernel<L_RCONTIG>, grid, 256, s, g);
  else
    launch(gemm_f32_dma_kernel<L_KCONTIG>, grid, 256, s, g);
}

}  // namespace hmx
