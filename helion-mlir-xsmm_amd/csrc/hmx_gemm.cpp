// Host side of the GEMM: the tile table and planner (hmx_gemm_plan), argument
// checks, the up-front A and B transposes, kernel selection and the split-K
// reduction launch (hmx_gemm). The kernels live in hmx_gemm_bf16_*.hip,
// hmx_gemm_dma.hip and hmx_gemm_f32.hip.
#include <algorithm>
#include <cstdlib>
#include <mutex>

#include "hmx_gemm_common.hpp"

// The workspace of hmx_gemm_noalloc: split-K partials and the transposed A and B
// of a launch, in device memory the library owns instead of memory a caller
// allocates. One copy per device, held until the process ends. Host code
// never uses this name as an address (on the host it names a stand-in, not
// device memory): it takes each device's address once, from
// hipGetSymbolAddress, and passes that.
static __device__ __align__(256) uint8_t scratch[HMX_GEMM_SCRATCH_BYTES];

namespace hmx {
namespace {

constexpr int64_t kScratchBytes = HMX_GEMM_SCRATCH_BYTES;

// The address of `scratch` on the current device, looked up once per device
// (with that device current) and kept.
int scratch_of_current_device(void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex lock;
  static void* addresses[kMaxDevices] = {};
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess)
    return set_error(HMX_ERR_HIP, "gemm_noalloc: hipGetDevice: %s", hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices)
    return set_error(HMX_ERR_INVALID, "gemm_noalloc: device %d is past the %d devices the scratch serves",
                     device, kMaxDevices);
  std::lock_guard<std::mutex> guard(lock);
  if (addresses[device] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return set_error(HMX_ERR_HIP, "gemm_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", device,
                       hipGetErrorString(err));
    addresses[device] = p;
  }
  *out = addresses[device];
  return HMX_OK;
}

struct TileChoice {
  int bm, bn, bk;
};

// Instantiated workgroup tiles, largest first.
constexpr TileChoice kBf16Tiles[] = {{256, 256, 64}, {128, 128, 64}};
constexpr TileChoice kF32Tiles[] = {{128, 128, 32}, {64, 64, 32}};
// The f32 tile long-K split-K products of whole 256 x 256 tiles take (see
// make_plan): one workgroup per CU reading each operand once.
constexpr TileChoice kF32Big = {256, 256, 32};
// The skinny kernel's plan (see skinny_shape).
constexpr TileChoice kSkinny = {32, 32, 64};

int layout_code(int b_layout) {
  switch (b_layout) {
    case HMX_B_ROW: return L_RCONTIG;
    case HMX_B_TRANS: return L_KCONTIG;
    case HMX_B_VNNI_PANELS: return L_VNNI_PANELS;
    case HMX_B_BLOCKED_VNNI: return L_BLOCKED_VNNI;
    case HMX_B_PANELS: return L_PANELS;
    case HMX_B_BLOCKED: return L_BLOCKED;
  }
  return -1;
}

struct Plan {
  TileChoice tile;
  int splits;
  int64_t k_chunk;
  int64_t workspace_bytes;
  // Row-major bf16 B is first transposed to [N, K] in the workspace (at
  // offset 0, bt_bytes long) when enough output rows reuse it: the K-contiguous
  // kernel path then reads it without register transposes.
  bool transpose_b;
  int64_t bt_bytes;
  // bf16 A stored [K, M] is first transposed to [M, K] in the workspace
  // (after the transposed B, at_bytes long), and the product is planned and
  // run as one of row-major A.
  bool transpose_a;
  int64_t at_bytes;
  // M <= 64 against B [N, K]: the skinny kernel (tile 32 x 32 x 64, no
  // split, no workspace).
  bool skinny;
};

// f32 products whose tiles fill at most a quarter of the CUs are bound by
// latency, not operand traffic: split K until the grid holds one workgroup
// per CU, each chunk keeping at least 4 K tiles, at most 16 splits (the
// partials are a few MiB at most), or as auto_splits says if that is more. HIP-graph replay on one box, 64 x 64
// tiles: 512^3 15.8 -> 12.3 us (4 splits, 1 before), 384 x 384 x 2048
// 53 -> 22 us (4, 1), 256 x 256 x 1024 27.6 -> 13.3 us (8, 1), 256 x 256 x
// 4096 32 -> 21 us (16, 4); 64 splits of 128 x 128 x 8192 took 37 us
// against 26 us for 16 (the reduction sums each output's partials in order).
int small_f32_splits(int64_t tiles, int64_t kt, int64_t outputs, int64_t max_ws, int cus) {
  int splits = 1;
  while (splits < 16 && tiles * splits * 2 <= cus && kt / (splits * 2) >= 4 &&
         (max_ws < 0 || (int64_t)splits * 2 * outputs * 4 <= max_ws))
    splits *= 2;
  return splits;
}

// Output rows from which a row-major bf16 B is transposed once up front.
constexpr int64_t kTransposeMinRows = 512;

// M, N and K from which a bf16 A stored [K, M] is transposed once up front,
// unless the environment sets HMX_GEMM_TRANSPOSE_A=0 (for comparison).
constexpr int64_t kTransposeAMin = 512;
bool transpose_a_enabled() {
  static const bool on = [] {
    const char* e = getenv("HMX_GEMM_TRANSPOSE_A");
    return !(e && e[0] == '0');
  }();
  return on;
}

// Split K while the grid holds fewer workgroups than there are CUs (bf16;
// for f32's smaller tiles, than four per CU), each chunk keeps at least 8 K
// tiles, and the partials (written and read again as f32) stay within a
// quarter of the operand traffic and the workspace limit. bf16 128 x 128
// tiles count one per CU: on a skinny 32 x 11008 x 4096 product four splits
// (344 workgroups) measure 26 us, eight 36 us.
int auto_splits(TileChoice tile, int64_t tiles, int64_t m, int64_t n, int64_t k, int64_t batch,
                int64_t esz, int64_t max_ws, int cus, bool fill = false) {
  const int64_t kt = ceil_div(k, tile.bk);
  const int64_t operand_bytes = batch * (m + n) * k * esz;
  const int64_t resident = (tile.bm == 256 || esz == 2 ? 1 : 4) * (int64_t)cus;
  int splits = 1;
  for (;;) {
    const int s2 = splits * 2;
    if (tiles * splits >= resident || kt / s2 < 8) break;
    const int64_t need = (int64_t)s2 * batch * m * n * 4;
    // The f32 partials' traffic (written once, read once) at most an eighth
    // of the operands'. With `fill`, bf16 128 x 128 tiles of products of at
    // least 2^30 multiply-adds, K in whole stages, also split while the grid
    // stays within one workgroup per CU, each chunk keeps 16 or more stages
    // and the partials move at most the operands' bytes: a grid of one such
    // workgroup per CU on a few CUs is latency-bound, and filling the CUs
    // pays for the partials (same box, unsplit -> split: 1024 x 1024 x 4096
    // 31.5 -> 21.5 us, 512 x 2048 x 8192 57 -> 28.5 us, 256 x 4000 x 4096
    // 33.7 -> 27.9 us, 768 x 768 x 3072 24.5 -> 20.5 us; a grid past one
    // workgroup per CU loses the four-stage ring: 256 x 11008 x 4096
    // 36 -> 44.5 us in two).
    const bool fills = fill && esz == 2 && tile.bm == 128 && k % tile.bk == 0 && kt / s2 >= 16 && tiles * s2 <= cus &&
                       (double)batch * m * n * k >= 1073741824.0 && need <= operand_bytes;
    if ((max_ws >= 0 && need > max_ws) || (2 * need > operand_bytes / 4 && !fills)) break;
    splits = s2;
  }
  return splits;
}

// Skinny products (at most 64 rows of row-major A against B [N, K], batch 1,
// K in whole 64-element stages) take the skinny kernel unless the caller
// asks for K splits or names another tile, or the environment sets
// HMX_GEMM_SKINNY=0 (for comparison). It reads B once with every CU
// streaming: 32 x 11008 x 4096 took 26 us as four splits of 128 x 128 tiles
// plus the reduction.
bool skinny_shape(int ab_dtype, int64_t m, int64_t k, int64_t batch, int trans_a, int b_layout,
                  int splits, int tile_m, int tile_n, int tile_k) {
  static const bool on = [] {
    const char* e = getenv("HMX_GEMM_SKINNY");
    return !(e && e[0] == '0');
  }();
  const bool no_tile = tile_m <= 0 && tile_n <= 0 && tile_k <= 0;
  const bool skinny_tile = tile_m == kSkinny.bm && tile_n == kSkinny.bn && tile_k == kSkinny.bk;
  return on && ab_dtype == HMX_DTYPE_BF16 && m >= 1 && m <= 64 && k >= 64 && k % 64 == 0 && batch == 1 &&
         !trans_a && b_layout == HMX_B_TRANS && splits <= 1 && (no_tile || skinny_tile);
}

bool dma_enabled();

// Whether an unsplit bf16 launch of this shape takes a direct-to-LDS kernel,
// which runs epilogue programs fused (select_kernel's rules with operands
// that keep 16-byte rows; B row-major or [N, K]).
bool program_fused_shape(const Plan& plan, bool bf16, int64_t m, int64_t n, int64_t k, int trans_a,
                         int b_layout) {
  const bool plain_b = b_layout == HMX_B_ROW || b_layout == HMX_B_TRANS;
  if (!bf16 || !plain_b || plan.splits > 1 || k <= 0 || plan.k_chunk % 32 != 0 || !dma_enabled())
    return false;
  const TileChoice t = plan.tile;
  const bool whole = m % t.bm == 0 && n % t.bn == 0 && plan.k_chunk % t.bk == 0 && k % t.bk == 0;
  const bool k64 = k % 64 == 0 && plan.k_chunk % 64 == 0;
  // Spans past 2^31 bytes take the register-staged kernel.
  const bool spans = m * k * 2 < INT32_MAX && n * k * 2 < INT32_MAX;
  if (!spans) return false;
  if (t.bm == 256) return trans_a ? whole : (whole || k64);
  return t.bm == 128 && !trans_a && k64;
}

// A plan is a pure function of the problem, the request (splits, tile) and
// the device's CU count. Passing a plan's own splits, tile and workspace
// back reproduces it exactly: a tile request that names an instantiated tile
// (or the skinny kernel's, or with two or more splits the f32 split-K tile)
// takes that tile, and the split count is rounded the same way both times.
int make_plan(int ab_dtype, int64_t m, int64_t n, int64_t k, int64_t batch, int trans_a,
              int b_layout, int splits, int64_t max_ws, int tile_m, int tile_n, int tile_k,
              int cus, int epilogue, Plan& plan) {
  const bool bf16 = ab_dtype == HMX_DTYPE_BF16;
  const bool program = epilogue == HMX_EPI_PROGRAM;
  // Epilogues the direct-to-LDS kernels finish in registers.
  const bool reg_epilogue =
      epilogue == HMX_EPI_IDENTITY || epilogue == HMX_EPI_RELU || epilogue == HMX_EPI_SILU;
  plan.skinny = !program &&
                skinny_shape(ab_dtype, m, k, batch, trans_a, b_layout, splits, tile_m, tile_n, tile_k);
  if (plan.skinny) {
    plan.tile = kSkinny;
    plan.splits = 1;
    plan.k_chunk = k;
    plan.transpose_b = plan.transpose_a = false;
    plan.bt_bytes = plan.at_bytes = 0;
    plan.workspace_bytes = 0;
    return HMX_OK;
  }
  // Transposed A read in place costs the 256 x 256 kernel two transposing
  // LDS reads per fragment (4096^3: 114-118 us against 94 for row-major A),
  // and other shapes of it take the register-staged kernel. A transpose up
  // front (one HBM read and write of A, 22.7 us for 4096 x 8192 under the
  // profiler, 5.9 TB/s) is cheaper from these sizes on (same box, in place -> transposed: 8192^2 x 4096 421 ->
  // 397 us, 2048^3 43 -> 34, 1024^3 22 -> 20, 3000^3 314 -> 212, 1000 x 4096
  // x 4096 203 -> 55, 4096 x 1000 x 4096 105 -> 62), except for whole 256 x
  // 256 tiles the in-place kernel takes with N up to 4096, where the two
  // measure level (4096^3: 120 us transposed).
  const bool ta_in_place = m % 256 == 0 && n % 256 == 0 && k % 64 == 0 && (m / 256) * (n / 256) >= cus &&
                           n <= 4096;
  plan.transpose_a = bf16 && trans_a && !program && batch == 1 && transpose_a_enabled() &&
                     (b_layout == HMX_B_ROW || b_layout == HMX_B_TRANS) && m >= kTransposeAMin &&
                     n >= kTransposeAMin && k >= kTransposeAMin && m * k * 2 < INT32_MAX && !ta_in_place;
  plan.at_bytes = plan.transpose_a ? ceil_div(m * k * 2, 256) * 256 : 0;
  if (plan.transpose_a && max_ws >= 0 && plan.at_bytes > max_ws) {
    plan.transpose_a = false;
    plan.at_bytes = 0;
  }
  if (plan.transpose_a) {
    trans_a = 0;
    if (max_ws >= 0) max_ws -= plan.at_bytes;
  }
  const TileChoice* table = bf16 ? kBf16Tiles : kF32Tiles;
  const int count = bf16 ? (int)(sizeof(kBf16Tiles) / sizeof(TileChoice))
                         : (int)(sizeof(kF32Tiles) / sizeof(TileChoice));
  // Packed B layouts are instantiated for the first tile only.
  const bool packed = b_layout != HMX_B_ROW && b_layout != HMX_B_TRANS;
  int pick = -1;
  // Whole 256 x 256 tiles of row-major A and an unpacked B: what the big f32
  // split-K tile serves.
  const bool big_shape = !packed && !trans_a && m % 256 == 0 && n % 256 == 0 && m > 0 && n > 0;
  if (!bf16 && (splits >= 2 || reg_epilogue) && tile_m == kF32Big.bm && tile_n == kF32Big.bn &&
      tile_k == kF32Big.bk && big_shape && k % kF32Big.bk == 0) {
    pick = -2;
  } else if (tile_m > 0 || tile_n > 0 || tile_k > 0) {
    for (int i = 0; i < count && pick < 0; ++i) {
      if ((tile_m <= 0 || table[i].bm <= tile_m) && (tile_n <= 0 || table[i].bn <= tile_n) &&
          (tile_k <= 0 || table[i].bk <= tile_k))
        pick = i;
    }
    if (pick < 0) pick = count - 1;
  } else {
    // The largest tile that still gives every CU a workgroup; else the smallest.
    pick = count - 1;
    for (int i = 0; i < count; ++i) {
      const int64_t tiles = ceil_div(m, table[i].bm) * ceil_div(n, table[i].bn) * batch;
      if (tiles >= cus) { pick = i; break; }
    }
    // f32: 128 x 128 tiles also when split-K fills the CUs with them (half the
    // operand traffic of 64 x 64 tiles); 64 x 64 tiles for products too small
    // for either (512^3: 16 workgroups of 128 x 128, too few K tiles to split).
    if (!bf16 && pick > 0) {
      const int64_t t128 = ceil_div(m, 128) * ceil_div(n, 128) * batch;
      if (t128 * auto_splits(table[0], t128, m, n, k, batch, 4, max_ws, cus) >= cus) pick = 0;
    }
    // Long-K bf16 products of whole 256 x 256 tiles that split-K can spread
    // over every CU take the big tile: it reads each operand once (half the
    // operand traffic of 128 x 128 tiles), and that traffic bounds them.
    const int64_t big_tiles = (m / 256) * (n / 256) * batch;
    const TileChoice big = bf16 ? table[0] : kF32Big;
    if (big_shape && k % big.bk == 0 && big_tiles < cus &&
        big_tiles * (splits > 0 ? splits
                                : auto_splits(big, big_tiles, m, n, k, batch, bf16 ? 2 : 4, max_ws, cus)) >=
            cus)
      pick = bf16 ? 0 : -2;
    // f32 products whose whole 256 x 256 tiles fill the CUs unsplit, with an
    // epilogue the kernel finishes in registers: the big tile in one pass
    // (4096^3: 1112 -> ~930 us against the 128 x 128 register-staged tile).
    if (!bf16 && splits <= 1 && reg_epilogue && big_shape && k % kF32Big.bk == 0 && k >= 8 * kF32Big.bk &&
        big_tiles >= cus)
      pick = -2;
  }
  if (packed && bf16) pick = 0;
  plan.tile = pick == -2 ? kF32Big : table[pick];
  const int64_t tiles = ceil_div(m, plan.tile.bm) * ceil_div(n, plan.tile.bn) * batch;
  const int64_t kt = ceil_div(k, plan.tile.bk);
  if (splits == 0) {
    splits = auto_splits(plan.tile, tiles, m, n, k, batch, bf16 ? 2 : 4, max_ws, cus, true);
    if (!bf16 && plan.tile.bm < 256 && tiles * 4 <= cus)
      splits = std::max(splits, small_f32_splits(tiles, kt, batch * m * n, max_ws, cus));
  }
  if (splits < 1) splits = 1;
  if (splits > 1) {
    // Whole K tiles per chunk; no empty chunks.
    plan.k_chunk = ceil_div(kt, splits) * plan.tile.bk;
    splits = (int)ceil_div(k, plan.k_chunk);
  } else {
    plan.k_chunk = k;
  }
  plan.splits = splits;
  // An epilogue program runs fused in the direct-to-LDS kernels; the others
  // write f32 products to the workspace (as one split) for the split-K
  // reduction to finish, so their plan holds those partials even unsplit.
  // The plan sees no pointers: it assumes operands that keep the 16-byte
  // alignment of whole rows, and reserves the partials for packed B (whose
  // panel widths it does not see) and for shapes no fused kernel takes.
  // hmx_gemm asks for them only when the launch stages the program.
  const int64_t partial_bytes =
      splits > 1 || (program && !program_fused_shape(plan, bf16, m, n, k, trans_a, b_layout))
          ? (int64_t)std::max(splits, 1) * batch * m * n * 4
          : 0;
  plan.bt_bytes = ceil_div(n * k * 2, 256) * 256;
  // The direct-to-LDS kernels read row-major B in place (256 x 256 tiles,
  // ragged M and N too, or transposed A on whole tiles; 128 x 128 tiles of
  // row-major A) when K chunks are whole 64-element stages; other bf16 shapes
  // with enough rows read it transposed up front.
  // (N % 8 == 0: the rows of a contiguous B keep the 16-byte alignment those
  // loads need.)
  const bool dma_reads_b = k % 64 == 0 && plan.k_chunk % 64 == 0 && n % 8 == 0 &&
                           ((plan.tile.bm == 256 && (!trans_a || (m % 256 == 0 && n % 256 == 0))) ||
                            (plan.tile.bm == 128 && !trans_a));
  plan.transpose_b = bf16 && b_layout == HMX_B_ROW && !dma_reads_b && batch == 1 &&
                     m >= kTransposeMinRows &&
                     n * k * 2 < INT32_MAX &&
                     (max_ws < 0 || plan.bt_bytes + partial_bytes <= max_ws);
  if (!plan.transpose_b) plan.bt_bytes = 0;
  plan.workspace_bytes = plan.bt_bytes + plan.at_bytes + partial_bytes;
  return HMX_OK;
}

// The direct-to-LDS bf16 kernel serves every case it can unless the
// environment sets HMX_GEMM_DMA=0 (which selects the register-staged kernel,
// for comparison).
bool dma_enabled() {
  static const bool on = [] {
    const char* e = getenv("HMX_GEMM_DMA");
    return !(e && e[0] == '0');
  }();
  return on;
}

// Whole rounds: a GEMM of more 256 x 256 tiles than CUs whose last round
// would keep at most half the CUs busy runs its first n1 tile columns (a whole
// number of rounds) as 256 x 256 tiles and the remaining columns as 256 x 128
// tiles, one round of half-size tiles, instead of a last round of full tiles
// on few CUs. Returns n1, or 0 when the split does not apply. The environment
// variable HMX_GEMM_ROUNDS=0 turns it off (for comparison).
int64_t whole_round_columns(int64_t tiles_m, int64_t tiles_n, int cus) {
  static const bool on = [] {
    const char* e = getenv("HMX_GEMM_ROUNDS");
    return !(e && e[0] == '0');
  }();
  const int64_t tiles = tiles_m * tiles_n, tail = tiles % cus;
  if (!on || tiles <= cus || tail == 0 || tail > cus / 2) return 0;
  if ((tiles - tail) % tiles_m != 0) return 0;
  return (tiles - tail) / tiles_m;
}

// The direct-to-LDS kernels finish C from registers for identity, ReLU and
// SiLU, which store bf16 C as 4-byte aligned column pairs; every other
// activation and epilogue programs go through their LDS-staged epilogue,
// which takes any alignment.
bool dma_direct_ok(const GemmArgs& g) {
  const bool direct = g.act == HMX_EPI_IDENTITY || g.act == HMX_EPI_RELU || g.act == HMX_EPI_SILU;
  const bool pair_ok = g.c_dtype != HMX_DTYPE_BF16 ||
                       (g.ldc % 2 == 0 && g.stride_c % 2 == 0 && g.stride_split % 2 == 0 &&
                        (((uintptr_t)g.c) & 3) == 0);
  return (!direct || pair_ok) && g.k_chunk % 32 == 0 && g.k > 0;
}

// The kernel families a launch can take.
enum class Kernel { SKINNY, SKINNY_TILES, DMA, DMA_TA, DMA128, BF16, F32_DMA, F32 };

// Whether a family runs epilogue programs fused (the direct-to-LDS bf16
// kernels, through their LDS-staged epilogue); the others leave them to the
// split-K reduction.
bool runs_programs(Kernel kind) {
  return kind == Kernel::DMA || kind == Kernel::DMA_TA || kind == Kernel::DMA128;
}

// The kernel family for the arguments `g` of a planned launch: the
// direct-to-LDS kernels wherever their shape, layout and alignment rules
// hold (HMX_GEMM_DMA=0 turns them off, for comparison), else the
// register-staged kernels.
Kernel select_kernel(const GemmArgs& g, const Plan& plan, int ab_dtype, int la, int lb, bool whole,
                     bool bytes_ok) {
  const bool aligned = g.a.vec && g.b.vec && bytes_ok;
  const bool plain_b = lb == L_KCONTIG || lb == L_RCONTIG;
  if (plan.skinny) return aligned && dma_enabled() ? Kernel::SKINNY : Kernel::SKINNY_TILES;
  if (ab_dtype == HMX_DTYPE_BF16) {
    const TileChoice t = plan.tile;
    const bool k64 = g.k % 64 == 0 && plan.k_chunk % 64 == 0;
    // Whole 256 x 256 tiles, or ragged M and N with K chunks of whole
    // 64-element stages and B K-contiguous or row-major.
    const bool dma_shape = aligned && (whole || (plain_b && k64));
    const bool ok = dma_direct_ok(g) && dma_enabled();
    if (t.bm == 256 && dma_shape && la == L_KCONTIG && (plain_b || gemm_bf16_dma_packed_ok(g, lb)) && ok)
      return Kernel::DMA;
    if (t.bm == 256 && la == L_RCONTIG && whole && aligned && plain_b && ok) return Kernel::DMA_TA;
    if (t.bm == 128 && la == L_KCONTIG && plain_b && aligned && k64 && ok) return Kernel::DMA128;
    return Kernel::BF16;
  }
  const bool guard = !(whole && aligned);
  // Unsplit, the f32 direct-to-LDS kernel finishes C itself: a register
  // activation, and bf16 C in 4-byte column pairs.
  const bool epi_ok = plan.splits > 1 || (dma_direct_ok(g) && (g.act == HMX_EPI_IDENTITY ||
                                                              g.act == HMX_EPI_RELU || g.act == HMX_EPI_SILU));
  if (plan.tile.bm == 256 && !guard && plain_b && g.k_chunk % 32 == 0 && epi_ok && dma_enabled())
    return Kernel::F32_DMA;
  return Kernel::F32;
}

// hmx_gemm and hmx_gemm_noalloc: checks, plan, launches. The workspace is
// `workspace` (workspace_bytes long) or, with `use_scratch`, the library's
// own per-device scratch array, looked up only when the plan needs workspace.
// Every workspace byte a launch reads it has written first (the A and B
// transposes and each split's whole partial tile), so nothing needs clearing
// between calls.
int gemm_impl(int ab_dtype, int c_dtype, const void* a, int64_t lda, int trans_a,
              const void* b, int64_t ldb, int b_layout, int64_t b_panel, int64_t b_kpad,
              void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int64_t batch,
              int64_t stride_a, int64_t stride_b, int64_t stride_c, const void* bias,
              const void* scale, const void* shift, int vec_dtype, int epilogue,
              float epilogue_arg, const hmx_program* program, int splits, void* workspace,
              int64_t workspace_bytes, bool use_scratch, int tile_m, int tile_n, int tile_k,
              void* stream) {
  HMX_REQUIRE(valid_dtype(ab_dtype) && valid_dtype(c_dtype), "gemm: unknown dtype");
  HMX_REQUIRE((bias == nullptr && scale == nullptr && shift == nullptr) || valid_dtype(vec_dtype),
              "gemm: unknown vector dtype %d", vec_dtype);
  // The allocation-free entry point runs kernels compiled at run time only
  // when an earlier call compiled them.
  const JitCompileOff no_compile(use_scratch);
  hmx_program prog;
  const int pst = check_epilogue("gemm", epilogue, program, &prog);
  if (pst != HMX_OK) return pst;
  const int lb = layout_code(b_layout);
  HMX_REQUIRE(lb >= 0, "gemm: unknown B layout %d", b_layout);
  HMX_REQUIRE(ab_dtype == HMX_DTYPE_BF16 || lb == L_KCONTIG || lb == L_RCONTIG ||
                  lb == L_BLOCKED || lb == L_PANELS,
              "gemm: VNNI layouts pair bf16 values; f32 B takes row-major, blocked or panel layouts");
  HMX_REQUIRE(!trans_a || lb == L_KCONTIG || lb == L_RCONTIG,
              "gemm: packed B layouts take a row-major A");
  HMX_REQUIRE(m >= 0 && n >= 0 && k >= 0 && batch >= 1, "gemm: invalid shape [%lld, %lld, %lld] x %lld",
              (long long)m, (long long)n, (long long)k, (long long)batch);
  HMX_REQUIRE(a && b && c, "gemm: null operand");
  HMX_REQUIRE(splits >= 0, "gemm: negative splits");
  const bool packed = lb != L_KCONTIG && lb != L_RCONTIG;
  if (!packed) {
    HMX_REQUIRE(lda >= (trans_a ? m : k) && lda >= 1, "gemm: lda %lld too small", (long long)lda);
    HMX_REQUIRE(ldb >= (lb == L_KCONTIG ? k : n) && ldb >= 1, "gemm: ldb %lld too small", (long long)ldb);
  } else {
    HMX_REQUIRE(b_kpad >= k && b_kpad % (lb == L_VNNI_PANELS ? 2 : 1) == 0,
                "gemm: packed K extent %lld does not cover K %lld", (long long)b_kpad, (long long)k);
    if (lb == L_BLOCKED_VNNI || lb == L_BLOCKED)
      HMX_REQUIRE(b_kpad % 32 == 0, "gemm: blocked K extent %lld is not a multiple of 32", (long long)b_kpad);
    if (lb == L_VNNI_PANELS || lb == L_PANELS)
      HMX_REQUIRE(b_panel >= 8 && b_panel % (lb == L_VNNI_PANELS ? 4 : 8) == 0,
                  "gemm: panel width %lld unsupported", (long long)b_panel);
  }
  HMX_REQUIRE(ldc >= n && ldc >= 1, "gemm: ldc %lld too small", (long long)ldc);
  if (m == 0 || n == 0) return HMX_OK;

  const DeviceShape dev = current_device_shape();
  Plan plan;
  const bool program_epi = epilogue == HMX_EPI_PROGRAM;
  make_plan(ab_dtype, m, n, k, batch, trans_a, b_layout, splits,
            use_scratch ? kScratchBytes : (workspace ? workspace_bytes : 0), tile_m, tile_n, tile_k, dev.cus,
            epilogue, plan);
  // A K-contiguous operand (row-major A, B [N, K]) spanning 2^31 bytes or
  // more is past the 32-bit offsets of the direct-to-LDS kernels' buffer
  // loads. Rather than run the register-staged kernel over the whole product,
  // such a product is cut into blocks of whole 256-row tiles of that operand
  // that each span less, every block a product of its own, unsplit, on the
  // rows (A) or columns (B) of C it owns, in order on the stream. Unsplit
  // products with a named epilogue only: split-K, an operand transposed up
  // front, an epilogue program and the allocation-free entry point keep the
  // register-staged kernel.
  if (!use_scratch && !program_epi && batch == 1 && !packed && !trans_a && plan.splits <= 1 &&
      !plan.transpose_b && !plan.transpose_a && k > 0) {
    const int64_t esz = dtype_bytes(ab_dtype), cb = dtype_bytes(c_dtype);
    // Rows of leading dimension ld whose span ((rows - 1) ld + k) esz stays
    // below 2^31 bytes, in whole 256-row tiles (0: not even one tile).
    auto fit = [&](int64_t ld) {
      const int64_t lim = (INT32_MAX - 1) / esz - k;
      return lim < 0 ? 0 : (lim / ld + 1) / 256 * 256;
    };
    auto part = [&](const void* pa, const void* pb, void* pc, int64_t rows, int64_t cols, const void* vb,
                    const void* vs, const void* vh) {
      return gemm_impl(ab_dtype, c_dtype, pa, lda, trans_a, pb, ldb, b_layout, b_panel, b_kpad, pc, ldc, rows,
                       cols, k, 1, 0, 0, 0, vb, vs, vh, vec_dtype, epilogue, epilogue_arg, program, 1, workspace,
                       workspace_bytes, false, tile_m, tile_n, tile_k, stream);
    };
    const int64_t step_a = fit(lda);
    if (((m - 1) * lda + k) * esz >= INT32_MAX && step_a > 0) {
      for (int64_t r = 0; r < m; r += step_a) {
        const int st = part((const char*)a + r * lda * esz, b, (char*)c + r * ldc * cb, std::min(step_a, m - r), n,
                            bias, scale, shift);
        if (st != HMX_OK) return st;
      }
      return HMX_OK;
    }
    const int64_t step_b = fit(ldb);
    if (lb == L_KCONTIG && ((n - 1) * ldb + k) * esz >= INT32_MAX && step_b > 0) {
      const int64_t vb = dtype_bytes(vec_dtype);
      auto at = [&](const void* v, int64_t col) { return v ? (const void*)((const char*)v + col * vb) : nullptr; };
      for (int64_t col = 0; col < n; col += step_b) {
        const int st = part(a, (const char*)b + col * ldb * esz, (char*)c + col * cb, m, std::min(step_b, n - col),
                            at(bias, col), at(scale, col), at(shift, col));
        if (st != HMX_OK) return st;
      }
      return HMX_OK;
    }
  }
  // Workspace is checked once the launch is known (below): a B transposed up
  // front (plan.bt_bytes), then an A transposed up front (plan.at_bytes), then
  // f32 partials for split-K or a staged epilogue program. The transposed
  // operands are read K-contiguous from the workspace.
  if (use_scratch && (plan.transpose_b || plan.transpose_a)) {
    const int st = scratch_of_current_device(&workspace);
    if (st != HMX_OK) return st;
    workspace_bytes = kScratchBytes;
  }
  const void* b_given = b;
  const int64_t ldb_given = ldb;
  int lb_run = lb;
  if (plan.transpose_b) {
    b = workspace;
    ldb = k;
    lb_run = L_KCONTIG;
  }
  const void* a_given = a;
  const int64_t lda_given = lda;
  if (plan.transpose_a) {
    a = workspace ? (const char*)workspace + plan.bt_bytes : nullptr;
    lda = k;
    trans_a = 0;
  }
  int64_t tiles_m = ceil_div(m, plan.tile.bm), tiles_n = ceil_div(n, plan.tile.bn);
  HMX_REQUIRE(tiles_m * tiles_n < ((int64_t)1 << 31) && batch < 65536 && plan.splits < 65536,
              "gemm: grid too large");

  const int64_t esz = dtype_bytes(ab_dtype);
  const int64_t vec_elems = 16 / esz;
  GemmArgs g{};
  const int la = trans_a ? L_RCONTIG : L_KCONTIG;
  g.a = Operand{a, lda, m, 0, 0,
                aligned16(a) && lda % vec_elems == 0 && (batch == 1 || stride_a % vec_elems == 0), 0};
  const int64_t b_rows = packed ? (lb == L_BLOCKED_VNNI || lb == L_BLOCKED ? ceil_div(n, 32) * 32
                                                                           : ceil_div(n, b_panel) * b_panel)
                                : n;
  g.b = Operand{b, ldb, b_rows, b_panel, b_kpad,
                aligned16(b) && (packed || ldb % vec_elems == 0) &&
                    (batch == 1 || stride_b % vec_elems == 0),
                0};
  // Bytes spanned by one batch slice of each operand: the buffer-load
  // range of the whole-tile path, which needs it below 2^31.
  const int64_t a_bytes = (trans_a ? (k - 1) * lda + m : (m - 1) * lda + k) * esz;
  const int64_t b_bytes =
      packed ? b_rows * b_kpad * esz : (lb_run == L_RCONTIG ? (k - 1) * ldb + n : (n - 1) * ldb + k) * esz;
  const bool bytes_ok = a_bytes < INT32_MAX && b_bytes < INT32_MAX;
  g.a.bytes = bytes_ok ? (int32_t)a_bytes : 0;
  g.b.bytes = bytes_ok ? (int32_t)b_bytes : 0;
  // Packed layouts read zeros (their padding) past N up to the padded extent;
  // columns past N are never stored.
  g.stride_a = stride_a;
  g.stride_b = stride_b;
  g.m = m;
  g.n = n;
  g.k = k;
  g.k_chunk = plan.k_chunk;
  g.cus = dev.cus;
  g.xcds = dev.xcds;
  g.tiles_m = (int)tiles_m;
  g.tiles_n = (int)tiles_n;
  g.bias = bias;
  g.scale = scale;
  g.shift = shift;
  g.vec_dtype = vec_dtype;
  g.act = epilogue;
  g.act_arg = epilogue_arg;
  g.prog = prog;
  g.c = c;
  g.c_dtype = c_dtype;
  g.ldc = ldc;
  g.stride_c = stride_c;
  g.stride_split = 0;

  bool whole = m % plan.tile.bm == 0 && n % plan.tile.bn == 0 &&
               plan.k_chunk % plan.tile.bk == 0 && k % plan.tile.bk == 0;
  bool guard = !(whole && g.a.vec && g.b.vec && bytes_ok);
  Kernel kind = select_kernel(g, plan, ab_dtype, la, lb_run, whole, bytes_ok);
  if (kind == Kernel::F32 && plan.tile.bm == 256 && plan.splits < 2) {
    // The unsplit 256 x 256 f32 tile runs on the direct-to-LDS kernel only
    // (aligned operands, an epilogue it finishes): otherwise the 128 x 128
    // tile, which needs no workspace either.
    const int st = make_plan(ab_dtype, m, n, k, batch, trans_a, b_layout, 1, -1, kF32Tiles[0].bm,
                             kF32Tiles[0].bn, kF32Tiles[0].bk, dev.cus, epilogue, plan);
    if (st != HMX_OK) return st;
    tiles_m = ceil_div(m, plan.tile.bm);
    tiles_n = ceil_div(n, plan.tile.bn);
    g.tiles_m = (int)tiles_m;
    g.tiles_n = (int)tiles_n;
    g.k_chunk = plan.k_chunk;
    whole = m % plan.tile.bm == 0 && n % plan.tile.bn == 0 && plan.k_chunk % plan.tile.bk == 0 &&
            k % plan.tile.bk == 0;
    guard = !(whole && g.a.vec && g.b.vec && bytes_ok);
    kind = select_kernel(g, plan, ab_dtype, la, lb_run, whole, bytes_ok);
  }
  // Split-K, and epilogue programs on kernels that do not run them fused:
  // the GEMM writes f32 partials ([splits, batch, M, N]) with the identity
  // epilogue, and the reduction applies bias, scale, shift and the epilogue.
  const bool staged = plan.splits > 1 || (program_epi && !runs_programs(kind));
  const int64_t need =
      plan.bt_bytes + plan.at_bytes + (staged ? (int64_t)std::max(plan.splits, 1) * batch * m * n * 4 : 0);
  const char* what = plan.splits > 1 ? "split-K"
                     : staged        ? "an epilogue program on these operands"
                                     : "the operand transpose";
  if (use_scratch && need > 0) {
    HMX_REQUIRE(need <= kScratchBytes,
                "gemm_noalloc: %s needs %lld bytes of workspace and the library's scratch holds %lld%s", what,
                (long long)need, (long long)kScratchBytes,
                plan.splits > 1 ? ": ask for fewer splits (splits = 0 plans within the scratch)" : "");
    if (workspace == nullptr) {
      const int st = scratch_of_current_device(&workspace);
      if (st != HMX_OK) return st;
      workspace_bytes = kScratchBytes;
    }
  }
  HMX_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need),
              "gemm: %s needs %lld workspace bytes, got %lld", what, (long long)need,
              (long long)(workspace ? workspace_bytes : 0));
  void* partials = workspace ? (char*)workspace + plan.bt_bytes + plan.at_bytes : nullptr;
  if (plan.transpose_a) {
    // A [K, M] -> [M, K] in the workspace, after the transposed B.
    launch_transpose16(a_given, (char*)workspace + plan.bt_bytes, k, m, lda_given, (hipStream_t)stream);
    const int st = check_launch("gemm A transpose");
    if (st != HMX_OK) return st;
  }
  if (plan.transpose_b) {
    // B [K, N] -> B^T [N, K] in the workspace; the GEMM then reads it K-contiguous.
    launch_transpose16(b_given, workspace, k, n, ldb_given, (hipStream_t)stream);
    const int st = check_launch("gemm B transpose");
    if (st != HMX_OK) return st;
  }
  if (staged) {
    // Split-K grids of one tile per batch slice share no operand data between
    // workgroups: each walks its K chunk from a stage of its own, so the
    // workgroups in flight read different K positions of their rows (bf16 bmm
    // [16, 256, 65536] x [16, 65536, 256]: 238 -> 208 us; the f32 one, MFMA-
    // bound, unchanged). Grids of several tiles keep the common walk, whose
    // shared A and B panels meet in L2 (a single tile row, whose workgroups
    // share only A, measured the same either way). HMX_GEMM_STAGGER=0 turns
    // it off (for comparison).
    static const bool stagger = [] {
      const char* e = getenv("HMX_GEMM_STAGGER");
      return !(e && e[0] == '0');
    }();
    g.k_stagger = stagger && plan.splits > 1 && tiles_m * tiles_n == 1;
    g.c = partials;
    g.c_dtype = HMX_DTYPE_F32;
    g.ldc = n;
    g.stride_c = m * n;
    g.stride_split = batch * m * n;
    g.bias = g.scale = g.shift = nullptr;
    g.act = HMX_EPI_IDENTITY;
    kind = select_kernel(g, plan, ab_dtype, la, lb_run, whole, bytes_ok);
  }

  const dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)plan.splits, (unsigned)batch);
  auto s = (hipStream_t)stream;
  switch (kind) {
    case Kernel::SKINNY:
      launch_gemm_bf16_skinny(g, s);
      break;
    case Kernel::SKINNY_TILES:
      // The skinny kernel's loads need the aligned, 2^31-bounded operands of
      // the direct-to-LDS kernels; otherwise the register-staged kernel runs
      // the same product on one 128 x 128 tile row.
      g.tiles_m = 1;
      g.tiles_n = (int)ceil_div(n, 128);
      launch_gemm_bf16(g, 128, la, lb_run, true, dim3((unsigned)g.tiles_n, 1, 1), s);
      break;
    case Kernel::DMA: {
      const int64_t n1 = whole && (lb_run == L_KCONTIG || lb_run == L_RCONTIG) && plan.splits == 1 &&
                                 batch == 1 && g.k_chunk % 64 == 0
                             ? whole_round_columns(tiles_m, tiles_n, dev.cus)
                             : 0;
      if (n1 > 0) {
        GemmArgs head = g;
        head.n = n1 * 256;
        head.tiles_n = (int)n1;
        // The rest: B rows, C columns and the column vectors from n1 * 256 on.
        const int64_t off = n1 * 256;
        GemmArgs rest = g;
        rest.n = n - off;
        rest.tiles_n = (int)(rest.n / 128);
        // B [N, K]: rows off..; B [K, N]: columns off.. of every row.
        rest.b.p = (const uint16_t*)g.b.p + (lb_run == L_RCONTIG ? off : off * g.b.ld);
        rest.b.rows = rest.n;
        rest.b.bytes = (int32_t)((lb_run == L_RCONTIG ? (k - 1) * g.b.ld + rest.n : (rest.n - 1) * g.b.ld + k) * 2);
        rest.c = (char*)g.c + off * dtype_bytes(g.c_dtype);
        const int64_t vb = off * dtype_bytes(vec_dtype);
        if (g.bias) rest.bias = (const char*)g.bias + vb;
        if (g.scale) rest.scale = (const char*)g.scale + vb;
        if (g.shift) rest.shift = (const char*)g.shift + vb;
        const unsigned head_blocks = (unsigned)(tiles_m * n1), rest_blocks = (unsigned)(tiles_m * rest.tiles_n);
        if (!launch_gemm_bf16_dma_rounds(head, rest, lb_run, head_blocks, rest_blocks, s)) {
          launch_gemm_bf16_dma(head, lb_run, dim3(head_blocks, 1, 1), s);
          launch_gemm_bf16_dma_narrow(rest, lb_run, dim3(rest_blocks, 1, 1), s);
        }
      } else {
        launch_gemm_bf16_dma(g, lb_run, grid, s);
      }
      break;
    }
    case Kernel::DMA_TA:
      launch_gemm_bf16_dma_ta(g, lb_run, grid, s);
      break;
    case Kernel::DMA128:
      launch_gemm_bf16_dma128(g, lb_run, grid, s);
      break;
    case Kernel::BF16:
      launch_gemm_bf16(g, plan.tile.bm, la, lb_run, guard, grid, s);
      break;
    case Kernel::F32_DMA:
      launch_gemm_f32_dma(g, lb, grid, s);
      break;
    case Kernel::F32:
      // The 256 x 256 f32 tile is planned only for row-major A, B [N, K] or
      // [K, N] and two or more splits: its kernel writes f32 partials with the
      // identity epilogue.
      if (plan.tile.bm == 256 && (plan.splits < 2 || la != L_KCONTIG))
        return set_error(HMX_ERR_INVALID, "gemm: internal f32 plan without split-K");
      launch_gemm_f32(g, plan.tile.bm, la, lb, guard, grid, s);
      break;
  }
  int st = check_launch("gemm");
  if (st != HMX_OK || !staged) return st;

  GemmArgs r = g;
  r.c = c;
  r.c_dtype = c_dtype;
  r.ldc = ldc;
  r.stride_c = stride_c;
  r.bias = bias;
  r.scale = scale;
  r.shift = shift;
  r.act = epilogue;
  const int64_t c_align = c_dtype == HMX_DTYPE_BF16 ? 8 : 16;
  const bool vec4 = n % 4 == 0 && ldc % 4 == 0 && stride_c % 4 == 0 && ((uintptr_t)c % c_align) == 0 &&
                    ((uintptr_t)partials % 16) == 0;
  launch_splitk_reduce((const float*)partials, plan.splits, batch, r, vec4, s);
  return check_launch("gemm split-K reduce");
}

}  // namespace
}  // namespace hmx

using namespace hmx;

extern "C" {

int hmx_gemm_plan(int ab_dtype, int64_t m, int64_t n, int64_t k, int64_t batch, int trans_a,
                  int b_layout, int splits, int64_t max_workspace_bytes, int tile_m,
                  int tile_n, int tile_k, int compute_units, int epilogue, int* out_splits,
                  int* out_tile_m, int* out_tile_n, int* out_tile_k, int64_t* out_workspace_bytes) {
  HMX_REQUIRE(valid_dtype(ab_dtype), "gemm_plan: unknown dtype %d", ab_dtype);
  HMX_REQUIRE(layout_code(b_layout) >= 0, "gemm_plan: unknown B layout %d", b_layout);
  HMX_REQUIRE(m >= 0 && n >= 0 && k >= 0 && batch >= 1, "gemm_plan: invalid shape");
  HMX_REQUIRE(splits >= 0, "gemm_plan: negative splits");
  HMX_REQUIRE(compute_units >= 0 && compute_units < 65536, "gemm_plan: invalid CU count %d", compute_units);
  const int cus = compute_units > 0 ? compute_units : current_device_shape().cus;
  Plan plan;
  HMX_REQUIRE(valid_activation(epilogue), "gemm_plan: unknown epilogue %d", epilogue);
  int st = make_plan(ab_dtype, m, n, k, batch, trans_a, b_layout, splits, max_workspace_bytes, tile_m,
                     tile_n, tile_k, cus, epilogue, plan);
  if (st != HMX_OK) return st;
  if (out_splits) *out_splits = plan.splits;
  if (out_tile_m) *out_tile_m = plan.tile.bm;
  if (out_tile_n) *out_tile_n = plan.tile.bn;
  if (out_tile_k) *out_tile_k = plan.tile.bk;
  if (out_workspace_bytes) *out_workspace_bytes = plan.workspace_bytes;
  return HMX_OK;
}

int hmx_gemm(int ab_dtype, int c_dtype, const void* a, int64_t lda, int trans_a,
             const void* b, int64_t ldb, int b_layout, int64_t b_panel, int64_t b_kpad,
             void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int64_t batch,
             int64_t stride_a, int64_t stride_b, int64_t stride_c, const void* bias,
             const void* scale, const void* shift, int vec_dtype, int epilogue,
             float epilogue_arg, const hmx_program* program, int splits, void* workspace,
             int64_t workspace_bytes, int tile_m, int tile_n, int tile_k, void* stream) {
  return gemm_impl(ab_dtype, c_dtype, a, lda, trans_a, b, ldb, b_layout, b_panel, b_kpad, c, ldc, m, n, k,
                   batch, stride_a, stride_b, stride_c, bias, scale, shift, vec_dtype, epilogue,
                   epilogue_arg, program, splits, workspace, workspace_bytes, false, tile_m, tile_n, tile_k,
                   stream);
}

int hmx_gemm_noalloc(int ab_dtype, int c_dtype, const void* a, int64_t lda, int trans_a,
                     const void* b, int64_t ldb, int b_layout, int64_t b_panel, int64_t b_kpad,
                     void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int64_t batch,
                     int64_t stride_a, int64_t stride_b, int64_t stride_c, const void* bias,
                     const void* scale, const void* shift, int vec_dtype, int epilogue,
                     float epilogue_arg, const hmx_program* program, int splits, int tile_m,
                     int tile_n, int tile_k, void* stream) {
  return gemm_impl(ab_dtype, c_dtype, a, lda, trans_a, b, ldb, b_layout, b_panel, b_kpad, c, ldc, m, n, k,
                   batch, stride_a, stride_b, stride_c, bias, scale, shift, vec_dtype, epilogue,
                   epilogue_arg, program, splits, nullptr, 0, true, tile_m, tile_n, tile_k, stream);
}

}  // extern "C"
