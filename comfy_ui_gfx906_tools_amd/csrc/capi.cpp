// C ABI of libqlinear.so (include/qlinear.h): argument checks, launch planning, error text.
// Counterpart of the reference's pybind11 layer (nodes/ComfyUI-Gfx906Int4/csrc/binding.cpp):
// the same checks, expressed as status codes plus a per-thread message instead of
// TORCH_CHECK exceptions; no tensor types cross this boundary.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include <vector>

#include "../../include/qlinear.h"
#include "common.hpp"
#include "launch.hpp"

using namespace qlinear;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return QL_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

const char* dtype_name(int dt) {
  switch (dt) {
    case QL_F32: return "float32";
    case QL_F16: return "float16";
    case QL_BF16: return "bfloat16";
    case QL_I32: return "int32";
    default: return "unknown";
  }
}

// CU count per device, queried once per device (callers may run on several threads).
int device_cus(int device, int* cus) {
  static std::mutex mu;
  static int cache[256] = {0};
  if (device < 0) {
    if (hipGetDevice(&device) != hipSuccess) return fail(QL_ERR_DEVICE, "hipGetDevice failed");
  }
  if (device >= 256) return fail(QL_ERR_DEVICE, "device index %d out of range", device);
  std::lock_guard<std::mutex> lock(mu);
  if (cache[device] == 0) {
    int v = 0;
    const hipError_t e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess || v <= 0)
      return fail(QL_ERR_DEVICE, "hipDeviceGetAttribute(MultiprocessorCount, %d): %s", device, hipGetErrorString(e));
    cache[device] = v;
  }
  *cus = cache[device];
  return QL_OK;
}

// ---- W4A16 launch plan ---------------------------------------------------------------------
// Tiles first go one per workgroup ("data-parallel"); when that leaves the last wave of a
// 1-workgroup-per-CU grid badly filled, the tiles of that last wave are cut into ksplit K
// pieces instead, chosen to minimise the modelled makespan (in tile-times).
// Workspace layout: [row scales: M fp32][column factors: N fp32][x16: M x K fp16][partial tiles: fp32]
constexpr int kMaxCutTiles = 1 << 16;

struct W4A16Plan {
  int cfg, BM, BN, tiles_m, tiles_n, stages, dp_tiles, ksplit, grid;
  bool prepass;    // stage x as row-scaled fp16
  bool col_scaled; // fp16 dequant: per-column power-of-two factors (computed unless the caller gives them)
  size_t off_row_scale, off_col_scale, off_x16, off_partial, total;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Kernel configurations: 0-3 are w4a16_gemm_kernel tiles of 256 / 128 / 64 / 16 rows x 256
// columns (4 waves side by side); 4-6 are the w4a16_tile256_kernel variants 0-2 (256 x 256
// tiles, whole tiles, K % 64 == 0); 7 is the VALU kernel for M <= 4 and 8 the MFMA kernel for
// M <= 16 (both read 16-bit x as is). Automatic choice: 7 for one row, 8 for up to 16 rows where
// it applies, then the smallest tile that covers M for M <= 128, else a 256 x 256 tile when its
// tiles fill every CU at least once, else 128-row tiles (whose last wave of tiles the planner may
// cut into K pieces).
constexpr int kCfgTile256 = 4;
constexpr int kCfgGemv = kCfgTile256 + kTile256Variants;  // 7: rows <= 4, VALU dot products
constexpr int kCfgSkinny = kCfgGemv + 1;                  // 8: rows <= 16, MFMA, K split in-workgroup
constexpr int kCfgLast = kCfgSkinny;
constexpr int kCfgTile256Auto = kCfgTile256 + 1;
bool is_tile256(int cfg) { return cfg >= kCfgTile256 && cfg < kCfgTile256 + kTile256Variants; }

// Tiles of the 256 x 256 kernel that run whole: every full round of CUs; the remaining tiles are
// cut into 128-row halves when their halves fit in one more round, else they run whole too.
int64_t tile256_whole(int64_t tiles, int cus) {
  const int64_t rem = tiles % cus;
  return (rem > 0 && 2 * rem <= cus) ? tiles - rem : tiles;
}

// K pieces per tile of the 256-column kernel, variant 1 only: an explicit splits >= 2, or (splits
// 0) enough pieces to give every CU one when the tiles alone fill at most a third of them, each
// piece at least kMinPieceStages stages of 64 K long (shorter ones spend more on the pipeline's
// fill and the partial round trip than they gain). Between a third and a half the K pieces do not
// pay for their partials (MI355X, M = 512, K = 3072, weights from HBM: N = 9216, 72 tiles, 3
// pieces 55.2 vs 60.5 us whole; N = 12288, 96 tiles, 2 pieces 63.1 vs 61.6 us whole), and those
// plans keep whole tiles and 128-row halves.
constexpr int kMinPieceStages = 4;
int tile256_pieces(int tiles, int stages, int splits, int cfg, int cus) {
  if (cfg != kCfgTile256Auto || splits == 1) return 1;
  if (splits >= 2) return std::min(splits, stages);
  if (3 * tiles > cus) return 1;
  return std::max(1, std::min(cus / tiles, stages / kMinPieceStages));
}

// 224-row tiles instead of 256 when the 256-row tiles make a single round that leaves CUs idle
// (more than half but not all of them busy) and 224-row tiles still fit one round with more CUs
// busy: each tile has 7/8 of the MFMA work (the same dequant). fc2 of the C2 pair (4608 x 3072):
// 216 -> 252 tiles on 256 CUs, 294.9 -> 289.3 us; C1 81.1 -> 79.6 us; the DiT's 4096-row img
// proj / fc2 (4096 x 3072): 192 -> 228 tiles, 0.5% faster. More CUs busy lower the power-limited
// clock, which takes back most of the gain. Results are bit-identical to the 256-row tiles.
bool tile224_fits(int64_t M, int64_t N, int cus) {
  const int64_t tn = (N + 255) / 256;
  const int64_t t256 = (M + 255) / 256 * tn, t224 = (M + 223) / 224 * tn;
  return 2 * t256 > cus && t256 < cus && t224 <= cus && t224 > t256;
}

// K pieces of the 4-wave kernel (configurations 0-3) with splits 0: when the last round of tiles
// fills the CUs badly (under 92%), its tiles are cut into as many K pieces as fit one round of
// workgroups, k = CUs / rem (at most 16 and the stage count); *dp = the tiles that run whole (the
// full rounds), the rest are cut. Returns 1 when nothing is cut (*dp = tiles). A second round of
// pieces costs more than its shorter pieces save (MI355X, K = 3072, N = 18432, weights from HBM,
// 72 tiles: 3 pieces 29.4 / 40.2 us at M = 64 / 128, 7 pieces in two rounds 36.9 / 61.2 us).
int four_wave_pieces(int tiles, int stages, int cus, int* dp) {
  *dp = tiles;
  if (stages < 2) return 1;
  const int waves = (tiles + cus - 1) / cus;
  if ((double)tiles / ((double)waves * cus) >= 0.92) return 1;
  const int whole = (tiles / cus) * cus;
  const int rem = tiles - whole;
  const int k = std::min(std::min(cus / rem, stages), 16);
  if (k < 2 || rem > kMaxCutTiles) return 1;
  *dp = whole;
  return k;
}

// 256 x 256 tiles once there are at least a quarter as many as CUs. Measured on MI355X (bf16 x via
// the fp16 staging, Flux DiT shapes): the 128-row kernel spends 1.6-2.2x the time per flop, so the
// 256 x 256 kernel wins even with most CUs idle (M=4096 N=3072 K=3072, 192 tiles: 80 vs 128 us;
// M=512 N=9216 K=3072, 72 tiles: 46 vs 103 us); with fewer tiles the 128-row kernel's K cuts spread
// the work over the CUs and win (M=512 N=3072, 24 tiles: K=3072 33 vs 40 us, K=12288 63 vs 139 us).
bool prefer_tile256(int64_t M, int64_t N, int64_t K, int cus) {
  if (K % 64 != 0) return false;
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  return 4 * tiles >= cus;
}

// Up to 4 rows of 16-bit activations go to the VALU kernel (configuration 7), read as they are.
// (An explicit K split, splits >= 2, needs the 4-wave kernel: the 256 x 256 kernel and the VALU
// kernel have none.)
bool gemv_fits(int x_dtype, int64_t M, int64_t K) {
  const int64_t mp = M <= 1 ? 1 : M <= 2 ? 2 : 4;  // rows the kernel instance handles
  return M <= kGemvMaxM && K <= kGemvMaxK && mp * K <= kGemvMaxMK && (x_dtype == QL_BF16 || x_dtype == QL_F16);
}

// Up to 16 rows of 16-bit activations, K % 128 == 0 and K <= 4096: the MFMA kernel for skinny M
// (configuration 8), also read as they are.
bool skinny_fits(int x_dtype, int64_t M, int64_t N, int64_t K) {
  return M <= kSkinnyMaxM && K % 128 == 0 && K <= kSkinnyMaxK && (N + 64) * (K / 2) < INT32_MAX &&
         (x_dtype == QL_BF16 || x_dtype == QL_F16);
}

// 16-column blocks per workgroup of the skinny kernel: the largest B whose grid is one round of
// workgroups over more than half the CUs, cus / 2 < ceil(N / 16B) <= cus; where none is, one block
// up to 8 rows and two above. A/B on MI355X (us per call, K = 3072 unless noted; B = 1 / 2 / 3):
// N = 10240, K = 4096, M = 16: - / 15.1 / 12.3, M = 4: 10.7 / 11.5 / 10.6; N = 12288, M = 16:
// - / 12.5 / 10.8; N = 6144, M = 4: 6.6 / 6.3 / 7.4; N = 3072, M = 4: 4.75 / 5.75 / -;
// N = 18432, M = 16: - / 17.4 / 19.3.
int skinny_blocks(int64_t M, int64_t N, int cus) {
  for (int b = kSkinnyMaxBlocks; b >= 1; --b) {
    const int64_t wg = (N + 16 * b - 1) / (16 * b);
    if (2 * wg > cus && wg <= cus) return b;
  }
  return M <= 8 ? 1 : 2;
}

// One row: the VALU kernel (8.8 us vs 10.6 us at K=4096 N=10240); 2-16 rows: the MFMA kernel
// (4 rows: 10.6 us vs 14.9 us; 16 rows: 12.3 us vs 22.6 us for the 16-row tile kernel, same
// shape).
// QL_W4A16_BF16_MFMA asks for the reference's bf16-rounded weights, which only the tile kernels
// compute; 7 and 8 use the exact codes and are skipped then.
int w4a16_cfg_for(int x_dtype, int64_t M, int64_t N, int64_t K, int splits, int flags, int cus) {
  // the direct kernels (7, 8) neither compute the bf16-rounded weights nor store row-scaled fp16
  const bool exact_ok =
      splits < 2 && !(flags & (QL_W4A16_BF16_MFMA | QL_W4A16_F16_ROWSCALED | QL_W4A16_GATED_RESIDUAL));
  if (exact_ok && M <= 1 && gemv_fits(x_dtype, M, K)) return kCfgGemv;
  if (exact_ok && skinny_fits(x_dtype, M, N, K)) return kCfgSkinny;
  if (exact_ok && gemv_fits(x_dtype, M, K)) return kCfgGemv;
  if (M <= 16) return 3;
  // 17-256 rows: the 4-wave kernel's 64- / 128-row tiles with K pieces. (The 256-column kernel's
  // 64- / 128-row tiles, configuration 5 forced, measured no faster with the weights streamed
  // from HBM: K = 4096, N = 10240, M = 64 28.7 vs 27.4 us, M = 128 35.4 vs 35.3 us.)
  if (M <= 64) return 2;
  if (M <= 128) return 1;
  if (splits < 2 && prefer_tile256(M, N, K, cus)) return kCfgTile256Auto;
  // Fewer 256 x 256 tiles than that: the 128-row tiles with K pieces (one round), unless that round
  // leaves more than a tenth of the CUs idle and the 256 x 256 tiles' own K pieces (one round, at
  // a quarter of the tiles) are at least 16 stages long; shorter pieces spend more on pipeline
  // fill and partials than the fuller round gains. Measured on MI355X, fp16 x, weights from HBM,
  // us 128-row round vs 256 x 256 pieces: K = 12288, N = 3072: M = 768 (84% of the CUs) 81.9 vs
  // 78.5, M = 1024 (75%) 104.8 vs 91.7, M = 512 (94%) 55.9 vs 57.9; K = 3072 (pieces of 7-10
  // stages): M = 768 38.3 vs 43.1, M = 1024 42.8 vs 45.4, N = 6144 M = 512 42.6 vs 44.8, and at
  // 94-100% M = 512 / 640 / 896 and N = 2048 M = 1024 30.6 / 31.2 / 37.0 / 32.4 vs 40.6 / 43.7 /
  // 41.6 / 46.9.
  if (splits == 0 && K % 64 == 0) {
    const W4A16Config& c = w4a16_config(1);
    const int tiles = (int)(((M + c.BM - 1) / c.BM) * ((N + c.BN - 1) / c.BN));
    int dp = tiles;
    const int k = four_wave_pieces(tiles, w4a16_steps(1, K), cus, &dp);
    const int64_t grid = dp + (int64_t)(tiles - dp) * k;
    const int t256 = (int)(((M + 255) / 256) * ((N + 255) / 256));
    const int stages = (int)(K / 64);
    const int k256 = tile256_pieces(t256, stages, 0, kCfgTile256Auto, cus);
    if (10 * grid < 9 * (int64_t)cus && stages / k256 >= 16) return kCfgTile256Auto;
  }
  return 1;
}

W4A16Plan plan_w4a16(int x_dtype, int64_t M, int64_t N, int64_t K, int splits, int flags, int cus) {
  W4A16Plan pl{};
  const int forced = (flags & QL_W4A16_CFG_MASK) >> QL_W4A16_CFG_SHIFT;
  pl.cfg = forced ? forced - 1 : w4a16_cfg_for(x_dtype, M, N, K, splits, flags, cus);
  const bool direct = pl.cfg == kCfgGemv || pl.cfg == kCfgSkinny;  // 16-bit x read as is
  pl.prepass = !direct && (x_dtype == QL_F32 || (x_dtype == QL_BF16 && !(flags & QL_W4A16_BF16_MFMA)));
  // the tile kernels round q * s to fp16 unless bf16 x meets bf16 MFMA; the direct kernels apply
  // the scale in fp32
  pl.col_scaled = !direct && !(x_dtype == QL_BF16 && (flags & QL_W4A16_BF16_MFMA));
  if (pl.cfg == kCfgGemv) {
    pl.BM = 4;
    pl.BN = 16;
    pl.stages = 1;
  } else if (pl.cfg == kCfgSkinny) {
    pl.BM = 16;
    pl.BN = 16 * skinny_blocks(M, N, cus);
    pl.stages = 1;
  } else if (is_tile256(pl.cfg)) {
    // variant 1 (configuration 5) takes the shortest tile height that covers M, 64 / 128 / 256,
    // or 224 rows where that fills more CUs in the same single round (tile224_fits)
    pl.BM = pl.cfg != kCfgTile256Auto ? 256 : M <= 64 ? 64 : M <= 128 ? 128 : 256;
    if (pl.cfg == kCfgTile256Auto && pl.BM == 256 && splits == 0 && tile224_fits(M, N, cus)) pl.BM = 224;
    pl.BN = 256;
    pl.stages = (int)(K / 64);
  } else {
    const W4A16Config& c = w4a16_config(pl.cfg);
    pl.BM = c.BM;
    pl.BN = c.BN;
    pl.stages = w4a16_steps(pl.cfg, K);  // K loop steps of the config's pipeline
  }
  pl.tiles_m = (int)((M + pl.BM - 1) / pl.BM);
  pl.tiles_n = (int)((N + pl.BN - 1) / pl.BN);
  const int tiles = pl.tiles_m * pl.tiles_n;
  pl.dp_tiles = tiles;
  pl.ksplit = 1;
  if (direct) {
    // one launch, no K split across workgroups
  } else if (is_tile256(pl.cfg)) {
    const int k = tile256_pieces(tiles, pl.stages, splits, pl.cfg, cus);
    if (k > 1) {  // every tile cut into k K pieces (variant 1)
      pl.dp_tiles = 0;
      pl.ksplit = k;
    } else {
      pl.dp_tiles = (splits == 1 || pl.BM != 256) ? tiles : (int)tile256_whole(tiles, cus);
    }
  } else if (splits >= 2 && tiles <= kMaxCutTiles) {
    pl.ksplit = std::min(splits, pl.stages);
    if (pl.ksplit >= 2) pl.dp_tiles = 0;
  } else if (splits == 0) {
    pl.ksplit = four_wave_pieces(tiles, pl.stages, cus, &pl.dp_tiles);
  }
  pl.grid = pl.dp_tiles + (tiles - pl.dp_tiles) * pl.ksplit;
  const size_t partial_bytes = (pl.dp_tiles < tiles && !direct && (!is_tile256(pl.cfg) || pl.ksplit > 1))
                                   ? (size_t)(tiles - pl.dp_tiles) * pl.ksplit * pl.BM * pl.BN * sizeof(float)
                                   : 0;
  pl.off_row_scale = 0;
  pl.off_col_scale = pl.off_row_scale + (pl.prepass ? align256((size_t)M * sizeof(float)) : 0);
  pl.off_x16 = pl.off_col_scale + (pl.col_scaled ? align256((size_t)N * sizeof(float)) : 0);
  pl.off_partial = pl.off_x16 + (pl.prepass ? align256((size_t)M * K * 2) : 0);
  pl.total = (pl.prepass || pl.col_scaled || partial_bytes) ? pl.off_partial + partial_bytes : 0;
  return pl;
}

int check_w4a16_shape(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N <= 0 || K < 32 || K % 32 != 0)
    return fail(QL_ERR_SHAPE, "expected x [M, K], w_q4 [N, K/2], w_scale [N, K/32] with K %% 32 == 0, K >= 32, N > 0; "
                "got M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  // the kernels address one tile's rows of x (up to 256 x K fp16) with 32-bit buffer offsets
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > (1 << 22))
    return fail(QL_ERR_SHAPE, "dimension too large: M=%lld N=%lld K=%lld (K <= 4194304)", (long long)M, (long long)N,
                (long long)K);
  return QL_OK;
}

// Argument checks of qlinear_w4a16_gemm that need no device: dtypes, shape, splits, flags.
int check_w4a16_args(int x_dtype, int out_dtype, const float* row_scale, int64_t M, int64_t N, int64_t K, int splits,
                     int flags) {
  if (x_dtype != QL_BF16 && x_dtype != QL_F16 && x_dtype != QL_F32)
    return fail(QL_ERR_DTYPE, "x dtype %s (%d) unsupported, expected bfloat16, float16 or float32", dtype_name(x_dtype),
                x_dtype);
  if (out_dtype != QL_F32 && out_dtype != QL_F16 && out_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "out dtype %s (%d) unsupported, expected float32/float16/bfloat16", dtype_name(out_dtype),
                out_dtype);
  if (int rc = check_w4a16_shape(M, N, K)) return rc;
  if (splits < 0 || splits > 64) return fail(QL_ERR_ARG, "splits must be in [0, 64], got %d", splits);
  if (flags & ~(QL_W4A16_BF16_MFMA | QL_W4A16_GELU_TANH | QL_W4A16_F16_ROWSCALED | QL_W4A16_GATED_RESIDUAL |
                QL_W4A16_CFG_MASK))
    return fail(QL_ERR_ARG, "unknown flags 0x%x", flags);
  if (flags & QL_W4A16_GATED_RESIDUAL) {
    const int forced = (flags & QL_W4A16_CFG_MASK) >> QL_W4A16_CFG_SHIFT;
    if (flags & QL_W4A16_F16_ROWSCALED)
      return fail(QL_ERR_ARG, "QL_W4A16_GATED_RESIDUAL and QL_W4A16_F16_ROWSCALED do not combine");
    if (forced && forced - 1 > kCfgTile256Auto)
      return fail(QL_ERR_ARG, "QL_W4A16_GATED_RESIDUAL runs on kernel configurations 0-%d, not %d", kCfgTile256Auto,
                  forced - 1);
  }
  if (flags & QL_W4A16_F16_ROWSCALED) {
    const int forced = (flags & QL_W4A16_CFG_MASK) >> QL_W4A16_CFG_SHIFT;
    if (out_dtype != QL_BF16)
      return fail(QL_ERR_ARG, "QL_W4A16_F16_ROWSCALED rounds to the logical output dtype bfloat16 (out dtype %s given)",
                  dtype_name(out_dtype));
    if ((flags & QL_W4A16_BF16_MFMA) || (x_dtype == QL_F16 && !row_scale))
      return fail(QL_ERR_ARG, "QL_W4A16_F16_ROWSCALED bounds each output row by its input row factor: it needs "
                  "float16 x with row_scale, or bfloat16 / float32 x on the fp16 staging route");
    if (forced && forced - 1 > 3 && forced - 1 != kCfgTile256Auto)
      return fail(QL_ERR_ARG, "QL_W4A16_F16_ROWSCALED runs on kernel configurations 0-3 and %d, not %d",
                  kCfgTile256Auto, forced - 1);
  }
  {
    const int forced = (flags & QL_W4A16_CFG_MASK) >> QL_W4A16_CFG_SHIFT;
    if (forced > kCfgLast + 1) return fail(QL_ERR_ARG, "flags: kernel configuration %d does not exist (0-%d)",
                                           forced - 1, kCfgLast);
    if (forced && is_tile256(forced - 1) && K % 64 != 0)
      return fail(QL_ERR_SHAPE, "kernel configuration %d needs K %% 64 == 0, got K=%lld", forced - 1, (long long)K);
    if (forced && is_tile256(forced - 1) && forced - 1 != kCfgTile256Auto && splits >= 2)
      return fail(QL_ERR_ARG, "kernel configuration %d runs whole tiles only (splits 0 or 1), got splits=%d",
                  forced - 1, splits);
    if (forced == kCfgGemv + 1 && !gemv_fits(x_dtype, M, K))
      return fail(QL_ERR_SHAPE, "kernel configuration %d needs M <= %d, K <= %d (K <= %d for M > 2) and "
                  "bfloat16/float16 x; got M=%lld K=%lld x %s", kCfgGemv, kGemvMaxM, kGemvMaxK, kGemvMaxMK / 4,
                  (long long)M, (long long)K, dtype_name(x_dtype));
    if (forced == kCfgSkinny + 1 && !skinny_fits(x_dtype, M, N, K))
      return fail(QL_ERR_SHAPE, "kernel configuration %d needs M <= %d, K %% 128 == 0, K <= %d and "
                  "bfloat16/float16 x; got M=%lld N=%lld K=%lld x %s", kCfgSkinny, kSkinnyMaxM, kSkinnyMaxK,
                  (long long)M, (long long)N, (long long)K, dtype_name(x_dtype));
    if ((forced == kCfgGemv + 1 || forced == kCfgSkinny + 1) && splits >= 2)
      return fail(QL_ERR_ARG, "kernel configuration %d has no K split (splits 0 or 1), got splits=%d", forced - 1,
                  splits);
  }
  if (row_scale && x_dtype != QL_F16)
    return fail(QL_ERR_ARG, "row_scale is only accepted with float16 x (from qlinear_rows_to_f16), got %s",
                dtype_name(x_dtype));
  return QL_OK;
}

// The reference's split-K choice for gemm_int4 (csrc/binding.cpp:21-43 of the reference): none
// when its 64 x 64 tiles fill two workgroups per CU, else about 2.4 rounds of workgroups, at most
// 8 splits and at least 8 k-tiles (of 128 K) per split.
constexpr int kW4A4MaxSplits = 8;
int w4a4_reference_splits(int64_t M, int64_t N, int64_t K, int cus) {
  const int64_t tiles = ((M + 63) / 64) * ((N + 63) / 64);
  const int64_t slots = (int64_t)cus * 2;
  if (tiles >= slots || tiles == 0) return 1;
  const int64_t k_tiles = (K / 32 + 3) / 4;
  const int64_t max_splits = std::min<int64_t>(kW4A4MaxSplits, std::max<int64_t>(1, k_tiles / 8));
  const int64_t wanted = (12 * slots + 5 * tiles - 1) / (5 * tiles);
  return (int)std::min(wanted, max_splits);
}

// The argument checks that do not depend on the call's pointers, for the host-only queries
// (workspace size, plan description, plan check): the row-scaled fp16 output is taken with its
// required bfloat16 logical dtype and, for fp16 x, a row_scale.
int check_w4a16_plan_args(int x_dtype, int64_t M, int64_t N, int64_t K, int splits, int flags) {
  static const float kSomeRowScale = 1.0f;
  const bool rowscaled = (flags & QL_W4A16_F16_ROWSCALED) != 0;
  return check_w4a16_args(x_dtype, rowscaled ? QL_BF16 : QL_F32, (rowscaled && x_dtype == QL_F16) ? &kSomeRowScale : nullptr,
                          M, N, K, splits, flags);
}

// ---- static scratch of the allocation-free W4A16 entry point ---------------------------------
// qlinear_w4a16_gemm_noalloc runs the same plan as qlinear_w4a16_gemm with this array as its
// workspace. Every GPU the library runs on holds its own copy (its code object's, loaded with the
// library) until the process ends. In host code `scratch` only names the symbol: its device
// address comes from hipGetSymbolAddress, once per device, with that device current, and only
// that address is passed to kernels.
constexpr size_t kNoAllocScratchBytes = QL_W4A16_NOALLOC_SCRATCH_BYTES;
__device__ __attribute__((aligned(256))) uint8_t scratch[kNoAllocScratchBytes];

int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[256] = {nullptr};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(QL_ERR_DEVICE, "hipGetDevice failed");
  if (device < 0 || device >= 256) return fail(QL_ERR_DEVICE, "device index %d out of range", device);
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(QL_ERR_DEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    addr[device] = p;
  }
  *out = addr[device];
  return QL_OK;
}

}  // namespace

extern "C" {

const char* qlinear_last_error(void) { return g_last_error.c_str(); }

int qlinear_abi_version(void) { return (4 << 16) | 0; }

size_t qlinear_w4a16_workspace_bytes(int x_dtype, int64_t M, int64_t N, int64_t K, int splits, int flags,
                                     int device) {
  // invalid arguments (a forced configuration that does not exist among them) plan nothing
  if (check_w4a16_plan_args(x_dtype, M, N, K, splits, flags) != QL_OK || M == 0) return 0;
  int cus = 0;
  if (device_cus(device, &cus) != QL_OK) return 0;
  return plan_w4a16(x_dtype, M, N, K, splits, flags, cus).total;
}

int qlinear_w4a16_auto_splits(int64_t M, int64_t N, int64_t K, int device) {
  if (int rc = check_w4a16_shape(M, N, K)) return -rc;
  int cus = 0;
  if (int rc = device_cus(device, &cus)) return -rc;
  if (M == 0) return 1;
  const W4A16Plan pl = plan_w4a16(QL_F16, M, N, K, 0, 0, cus);
  return pl.dp_tiles < pl.tiles_m * pl.tiles_n ? pl.ksplit : 1;
}

int qlinear_w4a16_gemm(int x_dtype, int out_dtype, const void* x, const float* row_scale, const void* w_q4,
                       const float* w_scale, const float* w_scale_kn, const float* col_scale, const void* bias, void* y,
                       const float* out_bound, float* out_row_scale, const ql_w4a16_residual* residual, int64_t M,
                       int64_t N, int64_t K, int splits, int flags, void* workspace, size_t workspace_bytes,
                       void* stream) {
  if (int rc = check_w4a16_args(x_dtype, out_dtype, row_scale, M, N, K, splits, flags)) return rc;
  if ((flags & QL_W4A16_F16_ROWSCALED) && M > 0 && (!out_bound || !out_row_scale))
    return fail(QL_ERR_ARG, "QL_W4A16_F16_ROWSCALED needs out_bound (qlinear_w4a16_out_bound) and out_row_scale [M]");
  const bool gated = (flags & QL_W4A16_GATED_RESIDUAL) != 0;
  if (gated != (residual != nullptr))
    return fail(QL_ERR_ARG, "residual must be given exactly when flags has QL_W4A16_GATED_RESIDUAL");
  if (gated && M > 0) {
    const size_t esz = out_dtype == QL_F32 ? 4 : 2;
    if (!residual->residual || !residual->gate)
      return fail(QL_ERR_ARG, "null residual / gate pointer in the gated residual");
    if (residual->gate_rows < 1 || residual->gate_rows > INT32_MAX)
      return fail(QL_ERR_ARG, "gate_rows must be in [1, 2^31), got %lld", (long long)residual->gate_rows);
    if (((uintptr_t)residual->residual | (uintptr_t)residual->gate) % esz)
      return fail(QL_ERR_ALIGN, "residual and gate must be aligned to their %zu-byte elements", esz);
  }
  if (M == 0) return ok();
  if (!x || !w_q4 || !w_scale || !y) return fail(QL_ERR_ARG, "null x / w_q4 / w_scale / y pointer");
  if (!aligned16(x) || !aligned16(w_q4))
    return fail(QL_ERR_ALIGN, "x and w_q4 must be 16-byte aligned (x=%p w_q4=%p)", x, w_q4);
  int cus = 0;
  if (int rc = device_cus(-1, &cus)) return rc;
  const W4A16Plan pl = plan_w4a16(x_dtype, M, N, K, splits, flags, cus);
  if (pl.total > 0 && (!workspace || workspace_bytes < pl.total))
    return fail(QL_ERR_WORKSPACE, "workspace of %zu bytes needed (M=%lld N=%lld K=%lld splits=%d flags=%d), got %zu at %p",
                pl.total, (long long)M, (long long)N, (long long)K, splits, flags, workspace_bytes, workspace);
  if (pl.total > 0 && !aligned16(workspace)) return fail(QL_ERR_ALIGN, "workspace must be 16-byte aligned");

  char* ws = (char*)workspace;
  W4A16Params p{};
  p.x = x;
  p.row_scale = row_scale;
  p.col_scale = nullptr;
  if (pl.col_scaled) {
    if (col_scale) {
      p.col_scale = col_scale;
    } else {
      float* cs = (float*)(ws + pl.off_col_scale);
      const hipError_t e = col_scales_launch(w_scale, cs, N, K / 32, (hipStream_t)stream);
      if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "column scale launch failed: %s", hipGetErrorString(e));
      p.col_scale = cs;
    }
  }
  if (pl.prepass) {
    float* rs = (float*)(ws + pl.off_row_scale);
    void* x16 = ws + pl.off_x16;
    const hipError_t e = rows_to_scaled_f16_launch(x_dtype, x, x16, rs, M, K, (hipStream_t)stream);
    if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "fp16 staging launch failed: %s", hipGetErrorString(e));
    p.x = x16;
    p.row_scale = rs;
  }
  p.wq = w_q4;
  // the tile kernels read the group-major copy when given; the direct kernels (7, 8) read whole
  // column rows of w_scale, which that layout already serves in long runs
  const bool kn = w_scale_kn && pl.cfg != kCfgGemv && pl.cfg != kCfgSkinny;
  p.ws = kn ? w_scale_kn : w_scale;
  p.scales_kn = kn ? 1 : 0;
  p.bias = bias;
  p.y = y;
  p.partial = pl.total ? (float*)(ws + pl.off_partial) : nullptr;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.out_dtype = (flags & QL_W4A16_F16_ROWSCALED) ? kBF16AsF16 : out_dtype;
  p.out_bound = out_bound;
  p.out_row_scale = out_row_scale;
  if (gated) {
    p.residual = residual->residual;
    p.gate = residual->gate;
    p.gate_rows = (int)residual->gate_rows;
  }
  p.act = (flags & QL_W4A16_GELU_TANH) ? kActGeluTanh : kActNone;
  p.cus = cus;
  p.tiles_m = pl.tiles_m;
  p.tiles_n = pl.tiles_n;
  p.stages = pl.stages;
  p.dp_tiles = pl.dp_tiles;
  p.ksplit = pl.ksplit;
  p.tile_rows = pl.BM;
  const bool bf16_mfma = x_dtype == QL_BF16 && !pl.prepass;
  const hipError_t e = pl.cfg == kCfgGemv     ? w4a16_gemv_launch(x_dtype == QL_BF16, p, (hipStream_t)stream)
                       : pl.cfg == kCfgSkinny ? w4a16_skinny_launch(x_dtype == QL_BF16, pl.BN / 16, p, (hipStream_t)stream)
                       : is_tile256(pl.cfg)
                           ? w4a16_tile256_launch(pl.cfg - kCfgTile256, bf16_mfma, p, (hipStream_t)stream)
                           : w4a16_launch(pl.cfg, bf16_mfma, p, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "w4a16 launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_w4a16_gemm_noalloc(int x_dtype, int out_dtype, const void* x, const float* row_scale, const void* w_q4,
                               const float* w_scale, const float* w_scale_kn, const float* col_scale, const void* bias,
                               void* y, const float* out_bound, float* out_row_scale,
                               const ql_w4a16_residual* residual, int64_t M, int64_t N, int64_t K, int splits,
                               int flags, void* stream) {
  // the checks qlinear_w4a16_gemm makes before planning, so the size check below sees a valid plan
  if (int rc = check_w4a16_args(x_dtype, out_dtype, row_scale, M, N, K, splits, flags)) return rc;
  if (M == 0) return ok();
  int cus = 0;
  if (int rc = device_cus(-1, &cus)) return rc;
  const size_t need = plan_w4a16(x_dtype, M, N, K, splits, flags, cus).total;
  if (need > kNoAllocScratchBytes)
    return fail(QL_ERR_WORKSPACE,
                "qlinear_w4a16_gemm_noalloc: this call needs %zu bytes of scratch (M=%lld N=%lld K=%lld splits=%d "
                "flags=%d), more than the %zu bytes of the static scratch; use qlinear_w4a16_gemm with a workspace",
                need, (long long)M, (long long)N, (long long)K, splits, flags, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_address(&ws)) return rc;
  }
  return qlinear_w4a16_gemm(x_dtype, out_dtype, x, row_scale, w_q4, w_scale, w_scale_kn, col_scale, bias, y, out_bound,
                            out_row_scale, residual, M, N, K, splits, flags, ws, need > 0 ? kNoAllocScratchBytes : 0,
                            stream);
}

int qlinear_w4a16_describe_plan(int x_dtype, int64_t M, int64_t N, int64_t K, int splits, int flags, int cus,
                                int* info) {
  if (!info) return fail(QL_ERR_ARG, "null info pointer");
  if (cus <= 0 || cus > 4096) return fail(QL_ERR_ARG, "cus must be in [1, 4096], got %d", cus);
  if (int rc = check_w4a16_plan_args(x_dtype, M, N, K, splits, flags)) return rc;
  const W4A16Plan pl = plan_w4a16(x_dtype, M, N, K, splits, flags, cus);
  info[0] = pl.cfg;
  info[1] = pl.BM;
  info[2] = pl.BN;
  info[3] = pl.dp_tiles;
  info[4] = pl.tiles_m * pl.tiles_n;
  info[5] = pl.ksplit;
  info[6] = pl.prepass ? 1 : 0;
  return ok();
}

int qlinear_check_launch_plan(int op, int x_dtype, int64_t M, int64_t N, int64_t K, int splits, int flags, int cus) {
  if (cus <= 0 || cus > 4096) return fail(QL_ERR_ARG, "cus must be in [1, 4096], got %d", cus);
  if (M <= 0) return fail(QL_ERR_ARG, "M must be > 0 for a plan check, got %lld", (long long)M);
  // One launch of `grid` workgroups: workgroup b runs tile (base + xcd_remap(b) / sub) of the
  // grouped order (rows m0 = tm * tile_rows + (g % sub) * (tile_rows / sub)), K piece g % pieces
  // (pieces > 1 only for cut tiles). Every (tile, piece, sub) must be covered exactly once over all
  // launches, every tile must start inside M and N, and a sub-tile that starts past M must be one
  // the kernel leaves by its early exit (allow_past_m).
  std::vector<int> seen;
  int tiles_m = 0, tiles_n = 0;
  auto fresh = [&](int tm_count, int tn_count, int per_tile) {
    tiles_m = tm_count;
    tiles_n = tn_count;
    seen.assign((size_t)tm_count * tn_count * per_tile, 0);
  };
  auto launch = [&](const char* what, int grid, int base, int sub, int pieces, int tile_rows, int tile_cols,
                    int group_m, bool allow_past_m) -> int {
    for (int b = 0; b < grid; ++b) {
      const int g = xcd_remap(b, grid);
      if (g < 0 || g >= grid)
        return fail(QL_ERR_SHAPE, "%s: xcd_remap(%d, %d) = %d is not a workgroup of the grid", what, b, grid, g);
      const int t = base + g / (sub * pieces);
      const int rest = g % (sub * pieces);
      if (t < 0 || t >= tiles_m * tiles_n)
        return fail(QL_ERR_SHAPE, "%s: workgroup %d maps to tile %d of %d", what, b, t, tiles_m * tiles_n);
      int tm = 0, tn = 0;
      tile_coords(t, tiles_m, tiles_n, group_m, tm, tn);
      if (tm < 0 || tm >= tiles_m || tn < 0 || tn >= tiles_n)
        return fail(QL_ERR_SHAPE, "%s: tile %d -> (%d, %d) outside %d x %d tiles", what, t, tm, tn, tiles_m, tiles_n);
      const int64_t m0 = (int64_t)tm * tile_rows + (int64_t)(rest % sub) * (tile_rows / sub);
      const int64_t n0 = (int64_t)tn * tile_cols;
      if (n0 >= N) return fail(QL_ERR_SHAPE, "%s: workgroup %d starts at column %lld >= N=%lld", what, b, (long long)n0,
                               (long long)N);
      if (m0 >= M && !allow_past_m)
        return fail(QL_ERR_SHAPE, "%s: workgroup %d starts at row %lld >= M=%lld", what, b, (long long)m0, (long long)M);
      const size_t slot = ((size_t)tm * tiles_n + tn) * (size_t)(sub * pieces) + (size_t)rest;
      if (slot >= seen.size() || seen[slot]++)
        return fail(QL_ERR_SHAPE, "%s: tile (%d, %d) part %d launched twice", what, tm, tn, rest);
    }
    return QL_OK;
  };
  auto all_seen = [&](const char* what) -> int {
    for (size_t i = 0; i < seen.size(); ++i)
      if (seen[i] != 1) return fail(QL_ERR_SHAPE, "%s: tile part %zu launched %d times", what, i, seen[i]);
    return QL_OK;
  };
  if (op == 0) {  // W4A16 (qlinear_w4a16_gemm's plan)
    if (int rc = check_w4a16_plan_args(x_dtype, M, N, K, splits, flags)) return rc;
    const W4A16Plan pl = plan_w4a16(x_dtype, M, N, K, splits, flags, cus);
    const int tiles = pl.tiles_m * pl.tiles_n;
    if (pl.cfg == kCfgGemv || pl.cfg == kCfgSkinny) {
      // column blocks per workgroup, no tiles along M (the direct kernels index columns only)
      if (pl.BM < M) return fail(QL_ERR_SHAPE, "direct kernel: %d rows per workgroup < M=%lld", pl.BM, (long long)M);
      return QL_OK;
    }
    if (pl.dp_tiles < 0 || pl.dp_tiles > tiles) return fail(QL_ERR_SHAPE, "dp_tiles %d of %d", pl.dp_tiles, tiles);
    if (is_tile256(pl.cfg) && (pl.BM != 256 || pl.ksplit > 1)) {
      // variant 1 with BM-row tiles: all whole, or all cut into ksplit K pieces (partials + reduce)
      if (pl.cfg != kCfgTile256Auto || (pl.BM != 64 && pl.BM != 128 && pl.BM != 224 && pl.BM != 256))
        return fail(QL_ERR_SHAPE, "tile256 rows: configuration %d with %d-row tiles", pl.cfg, pl.BM);
      if (pl.BM == 224 && (pl.ksplit != 1 || pl.dp_tiles != tiles || tiles > cus))
        return fail(QL_ERR_SHAPE, "tile256 rows: 224-row tiles are one round of whole tiles (%d of %d, ksplit %d)",
                    pl.dp_tiles, tiles, pl.ksplit);
      if (pl.ksplit > 1 && pl.dp_tiles != 0)
        return fail(QL_ERR_SHAPE, "tile256 rows: %d whole tiles beside K pieces", pl.dp_tiles);
      if (pl.ksplit < 1 || pl.ksplit > pl.stages)
        return fail(QL_ERR_SHAPE, "tile256 rows: ksplit %d outside [1, %d stages]", pl.ksplit, pl.stages);
      fresh(pl.tiles_m, pl.tiles_n, pl.ksplit);
      if (int rc = launch("tile256 rows whole", pl.dp_tiles, 0, 1, 1, pl.BM, 256, kTile256GroupM, false)) return rc;
      if (int rc = launch("tile256 rows cut", (tiles - pl.dp_tiles) * pl.ksplit, pl.dp_tiles, 1, pl.ksplit, pl.BM, 256,
                          kTile256GroupM, false))
        return rc;
      if (pl.ksplit > 1) {
        const size_t partial_slots =
            pl.total >= pl.off_partial ? (pl.total - pl.off_partial) / ((size_t)pl.BM * pl.BN * 4) : 0;
        if (partial_slots < (size_t)tiles * pl.ksplit)
          return fail(QL_ERR_SHAPE, "tile256 rows: workspace holds %zu partial tiles, the launch writes %d",
                      partial_slots, tiles * pl.ksplit);
      }
      return all_seen("tile256 rows");
    }
    if (is_tile256(pl.cfg)) {
      // whole 256 x 256 tiles, then the rest as 128-row halves (a half wholly past M exits early)
      fresh(pl.tiles_m, pl.tiles_n, 2);
      // whole tiles occupy both halves of their slot
      for (int b = 0; b < pl.dp_tiles; ++b) {
        const int g = xcd_remap(b, pl.dp_tiles);
        int tm = 0, tn = 0;
        tile_coords(g, tiles_m, tiles_n, kTile256GroupM, tm, tn);
        if ((int64_t)tm * 256 >= M || (int64_t)tn * 256 >= N)
          return fail(QL_ERR_SHAPE, "tile256 whole: workgroup %d at (%d, %d) starts outside M x N", b, tm, tn);
        const size_t slot = ((size_t)tm * tiles_n + tn) * 2;
        if (seen[slot]++ || seen[slot + 1]++) return fail(QL_ERR_SHAPE, "tile256 whole: tile (%d, %d) twice", tm, tn);
      }
      if (int rc = launch("tile256 halves", 2 * (tiles - pl.dp_tiles), pl.dp_tiles, 2, 1, 256, 256, kTile256GroupM, true))
        return rc;
      return all_seen("tile256");
    }
    // configurations 0-3: whole tiles, then the cut tiles as ksplit K pieces each
    fresh(pl.tiles_m, pl.tiles_n, 1);
    if (int rc = launch("w4a16 whole", pl.dp_tiles, 0, 1, 1, pl.BM, pl.BN, kW4A16GroupM, false)) return rc;
    if (pl.dp_tiles < tiles) {
      if (pl.ksplit < 1 || pl.ksplit > pl.stages)
        return fail(QL_ERR_SHAPE, "ksplit %d outside [1, %d stages]", pl.ksplit, pl.stages);
      std::vector<int> whole = seen;
      seen.assign((size_t)tiles * pl.ksplit, 0);
      for (int i = 0; i < tiles; ++i)  // a whole tile stands for all its pieces
        for (int q = 0; q < pl.ksplit; ++q) seen[(size_t)i * pl.ksplit + q] = whole[i];
      // the cut launch numbers its pieces tile-major: piece = g - (t - dp) * ksplit
      for (int b = 0; b < (tiles - pl.dp_tiles) * pl.ksplit; ++b) {
        const int g = xcd_remap(b, (tiles - pl.dp_tiles) * pl.ksplit);
        const int t = pl.dp_tiles + g / pl.ksplit, piece = g % pl.ksplit;
        int tm = 0, tn = 0;
        tile_coords(t, tiles_m, tiles_n, kW4A16GroupM, tm, tn);
        if ((int64_t)tm * pl.BM >= M || (int64_t)tn * pl.BN >= N || t >= tiles)
          return fail(QL_ERR_SHAPE, "w4a16 cut: workgroup %d at tile %d (%d, %d) starts outside M x N", b, t, tm, tn);
        const int s0 = (int)((long long)piece * pl.stages / pl.ksplit), s1 = (int)((long long)(piece + 1) * pl.stages / pl.ksplit);
        if (s0 < 0 || s1 < s0 || s1 > pl.stages) return fail(QL_ERR_SHAPE, "w4a16 cut: piece %d range [%d, %d)", piece, s0, s1);
        const size_t slot = ((size_t)tm * tiles_n + tn) * pl.ksplit + piece;
        if (seen[slot]++) return fail(QL_ERR_SHAPE, "w4a16 cut: tile (%d, %d) piece %d twice", tm, tn, piece);
      }
      const size_t partial_slots = pl.total >= pl.off_partial ? (pl.total - pl.off_partial) / ((size_t)pl.BM * pl.BN * 4) : 0;
      if (partial_slots < (size_t)(tiles - pl.dp_tiles) * pl.ksplit)
        return fail(QL_ERR_SHAPE, "w4a16 cut: workspace holds %zu partial tiles, the launch writes %d", partial_slots,
                    (tiles - pl.dp_tiles) * pl.ksplit);
    }
    return all_seen("w4a16");
  }
  if (op == 1) {  // W8A8 (qlinear_w8a8_gemm's choice)
    if (K < 64 || K % 64 != 0 || N <= 0) return fail(QL_ERR_SHAPE, "W8A8 needs K %% 64 == 0, N > 0");
    const bool big = M > 128 && K * kW8A8Tile256 <= INT32_MAX;
    const int cfg = M <= 16 ? 3 : M <= 64 ? 2 : 1;
    const int BM = big ? kW8A8Tile256 : w8a8_config(cfg).BM, BN = big ? kW8A8Tile256 : w8a8_config(cfg).BN;
    fresh((int)((M + BM - 1) / BM), (int)((N + BN - 1) / BN), 1);
    if (int rc = launch("w8a8", tiles_m * tiles_n, 0, 1, 1, BM, BN, big ? kW8A8T256GroupM : kW8A8GroupM, false)) return rc;
    return all_seen("w8a8");
  }
  if (op == 2) {  // W4A4 / block-32 int8 (128 x 128 tiles; split-K as grid.y)
    if (K < 32 || K % 32 != 0 || N <= 0 || splits < 1 || splits > kW4A4MaxSplits)
      return fail(QL_ERR_SHAPE, "W4A4 needs K %% 32 == 0, N > 0 and splits in [1, %d]", kW4A4MaxSplits);
    fresh((int)((M + 127) / 128), (int)((N + 127) / 128), 1);
    if (int rc = launch("w4a4", tiles_m * tiles_n, 0, 1, 1, 128, 128, kW4A4GroupM, false)) return rc;
    const int k_tiles = (int)((K / 32 + 3) / 4), per = (k_tiles + splits - 1) / splits;
    if (splits > 1 && (int64_t)per * splits < k_tiles) return fail(QL_ERR_SHAPE, "w4a4 splits miss k-tiles");
    return all_seen("w4a4");
  }
  return fail(QL_ERR_ARG, "op must be 0 (W4A16), 1 (W8A8) or 2 (W4A4), got %d", op);
}

int qlinear_w4a16_out_bound(const void* w_q4, const float* w_scale, const void* bias, int bias_dtype, int64_t N,
                            int64_t K, float* bound, void* stream) {
  if (N <= 0 || K < 32 || K % 32 != 0 || N > INT32_MAX / 2 || K > (1 << 22))
    return fail(QL_ERR_SHAPE, "expected w_q4 [N, K/2], w_scale [N, K/32] with K %% 32 == 0, N > 0; got N=%lld K=%lld",
                (long long)N, (long long)K);
  if (bias && bias_dtype != QL_F32 && bias_dtype != QL_F16 && bias_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "bias dtype %s (%d) unsupported", dtype_name(bias_dtype), bias_dtype);
  if (!w_q4 || !w_scale || !bound) return fail(QL_ERR_ARG, "null w_q4 / w_scale / bound pointer");
  if (!aligned16(w_q4)) return fail(QL_ERR_ALIGN, "w_q4 must be 16-byte aligned");
  const hipError_t e = w4a16_out_bound_launch(w_q4, w_scale, bias, bias_dtype, N, K, bound, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "w4a16_out_bound launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_w4a16_col_scales(const float* w_scale, float* col_scale, int64_t N, int64_t K, void* stream) {
  if (N < 0 || K < 32 || K % 32 != 0 || N > INT32_MAX / 2 || K > (1 << 22))
    return fail(QL_ERR_SHAPE, "expected w_scale [N, K/32] with K %% 32 == 0, 32 <= K <= 4194304; got N=%lld K=%lld",
                (long long)N, (long long)K);
  if (N == 0) return ok();
  if (!w_scale || !col_scale) return fail(QL_ERR_ARG, "null w_scale / col_scale pointer");
  const hipError_t e = col_scales_launch(w_scale, col_scale, N, K / 32, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "col_scales launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_w4a16_scales_kn(const float* w_scale, float* w_scale_kn, int64_t N, int64_t K, void* stream) {
  if (N < 0 || K < 32 || K % 32 != 0 || N > INT32_MAX / 2 || K > (1 << 22) || N * (K / 32) > INT32_MAX / 4)
    return fail(QL_ERR_SHAPE, "expected w_scale [N, K/32] with K %% 32 == 0, 32 <= K <= 4194304, N * K / 8 < 2^31; "
                "got N=%lld K=%lld", (long long)N, (long long)K);
  if (N == 0) return ok();
  if (!w_scale || !w_scale_kn) return fail(QL_ERR_ARG, "null w_scale / w_scale_kn pointer");
  const hipError_t e = scales_kn_launch(w_scale, w_scale_kn, N, K / 32, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "scales_kn launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_rows_to_f16(int x_dtype, const void* x, void* x16, float* row_scale, int64_t M, int64_t K,
                        void* stream) {
  if (x_dtype != QL_F32 && x_dtype != QL_F16 && x_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "unsupported dtype %s (%d), expected float32/float16/bfloat16", dtype_name(x_dtype),
                x_dtype);
  if (M < 0 || K <= 0 || K % 8 != 0 || K > INT32_MAX / 2 || M > INT32_MAX)
    return fail(QL_ERR_SHAPE, "x must be [M, K] with K %% 8 == 0, got [%lld, %lld]", (long long)M, (long long)K);
  if (M == 0) return ok();
  if (!x || !x16 || !row_scale) return fail(QL_ERR_ARG, "null x / x16 / row_scale pointer");
  if (!aligned16(x) || !aligned16(x16)) return fail(QL_ERR_ALIGN, "x and x16 must be 16-byte aligned");
  const hipError_t e = rows_to_scaled_f16_launch(x_dtype, x, x16, row_scale, M, K, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "rows_to_f16 launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_quantize_int4(int x_dtype, int rule, const void* x, void* packed, float* scale, int64_t rows,
                          int64_t K, void* stream) {
  if (x_dtype != QL_F32 && x_dtype != QL_F16 && x_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "unsupported dtype %s (%d), expected float32/float16/bfloat16", dtype_name(x_dtype),
                x_dtype);
  if (rule != 0 && rule != 1) return fail(QL_ERR_ARG, "rule must be 0 (amax / 7) or 1 (amax * (1/7)), got %d", rule);
  if (rows < 0 || K < 32 || K % 32 != 0)
    return fail(QL_ERR_SHAPE, "x must be [rows, K] with K %% 32 == 0, got [%lld, %lld]", (long long)rows, (long long)K);
  if (rows == 0) return ok();
  if (!x || !packed || !scale) return fail(QL_ERR_ARG, "null x / packed / scale pointer");
  if (!aligned16(x) || !aligned16(packed)) return fail(QL_ERR_ALIGN, "x and packed must be 16-byte aligned");
  const hipError_t e = quantize_int4_launch(x_dtype, rule, x, packed, scale, rows, K, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "quantize_int4 launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_repack_q4_0(const void* raw, int8_t* packed, float* scale, int64_t rows, int64_t K, void* stream) {
  if (rows < 0 || K < 32 || K % 32 != 0)
    return fail(QL_ERR_SHAPE, "Q4_0 weight must be [rows, K] with K %% 32 == 0, got [%lld, %lld]", (long long)rows,
                (long long)K);
  if (rows == 0) return ok();
  if (!raw || !packed || !scale) return fail(QL_ERR_ARG, "null raw / packed / scale pointer");
  if (((uintptr_t)raw & 1) || !aligned16(packed) || ((uintptr_t)scale & 3))
    return fail(QL_ERR_ALIGN, "raw must be 2-byte, packed 16-byte and scale 4-byte aligned");
  const hipError_t e = repack_q4_0_launch(raw, packed, scale, rows * (K / 32), (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "repack_q4_0 launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_quantize_int8_per_token(int x_dtype, const void* x, int8_t* q, float* scale, int64_t M, int64_t K,
                                    void* stream) {
  if (x_dtype != QL_F32 && x_dtype != QL_F16 && x_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "unsupported dtype %s (%d), expected float32/float16/bfloat16", dtype_name(x_dtype),
                x_dtype);
  if (M < 0 || K <= 0 || K > INT32_MAX / 2)
    return fail(QL_ERR_SHAPE, "x must be [M, K] with K > 0, got [%lld, %lld]", (long long)M, (long long)K);
  if (M == 0) return ok();
  if (M > INT32_MAX) return fail(QL_ERR_SHAPE, "M=%lld too large", (long long)M);
  if (!x || !q || !scale) return fail(QL_ERR_ARG, "null x / q / scale pointer");
  const hipError_t e = quantize_int8_per_token_launch(x_dtype, x, q, scale, M, K, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "quantize_int8_per_token launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_w8a8_gemm(int out_dtype, const int8_t* xq, const float* x_scale, const int8_t* wq, const float* w_scale,
                      const void* bias, void* y, int64_t M, int64_t N, int64_t K, void* stream) {
  if (out_dtype != QL_F32 && out_dtype != QL_F16 && out_dtype != QL_BF16 && out_dtype != QL_I32)
    return fail(QL_ERR_DTYPE, "out dtype %s (%d) unsupported, expected float32/float16/bfloat16/int32",
                dtype_name(out_dtype), out_dtype);
  if (M < 0 || N <= 0 || K < 64 || K % 64 != 0 || M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2)
    return fail(QL_ERR_SHAPE, "expected xq [M, K], wq [N, K] with K %% 64 == 0, N > 0; got M=%lld N=%lld K=%lld",
                (long long)M, (long long)N, (long long)K);
  if (M == 0) return ok();
  if (!xq || !wq || !y) return fail(QL_ERR_ARG, "null xq / wq / y pointer");
  if (out_dtype != QL_I32 && (!x_scale || !w_scale)) return fail(QL_ERR_ARG, "null x_scale / w_scale pointer");
  if (!aligned16(xq) || !aligned16(wq)) return fail(QL_ERR_ALIGN, "xq and wq must be 16-byte aligned");
  // M > 128: the 256 x 256-tile kernel (32-bit buffer offsets: 256 * K bytes per operand tile);
  // skinny M: the 16 / 64 / 128-row tiles
  const bool big = M > 128 && K * kW8A8Tile256 <= INT32_MAX;
  const int cfg = M <= 16 ? 3 : M <= 64 ? 2 : 1;
  const W8A8Config& c = w8a8_config(cfg);
  const int BM = big ? kW8A8Tile256 : c.BM, BN = big ? kW8A8Tile256 : c.BN;
  W8A8Params p{};
  p.xq = xq;
  p.sx = x_scale;
  p.wq = wq;
  p.sw = w_scale;
  p.bias = bias;
  p.y = y;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.out_dtype = out_dtype;
  p.tiles_m = (int)((M + BM - 1) / BM);
  p.tiles_n = (int)((N + BN - 1) / BN);
  p.stages = (int)((K + 255) / 256);
  const hipError_t e = big ? w8a8_tile256_launch(p, (hipStream_t)stream)
                           : w8a8_launch(cfg, p, p.tiles_m * p.tiles_n, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "w8a8 launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_adaln_modulate(int out_kind, int x_dtype, const void* x, int mod_dtype, const void* shift,
                           const void* scale, void* out, float* row_scale, int64_t M, int64_t K, float eps,
                           void* stream) {
  if (out_kind != QL_OPERAND_F16_ROWSCALED && out_kind != QL_OPERAND_PLAIN && out_kind != QL_OPERAND_I8_PER_TOKEN)
    return fail(QL_ERR_ARG, "out_kind must be QL_OPERAND_F16_ROWSCALED, QL_OPERAND_PLAIN or QL_OPERAND_I8_PER_TOKEN, got %d",
                out_kind);
  if (x_dtype != QL_F32 && x_dtype != QL_F16 && x_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "x dtype %s (%d) unsupported, expected float32/float16/bfloat16", dtype_name(x_dtype),
                x_dtype);
  if (mod_dtype != QL_F32 && mod_dtype != QL_F16 && mod_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "shift/scale dtype %s (%d) unsupported, expected float32/float16/bfloat16",
                dtype_name(mod_dtype), mod_dtype);
  if (M < 0 || M > INT32_MAX || K <= 0 || K % 8 != 0 || K > 16384)
    return fail(QL_ERR_SHAPE, "x must be [M, K] with K %% 8 == 0 and K <= 16384, got [%lld, %lld]", (long long)M,
                (long long)K);
  if (!(eps >= 0.0f)) return fail(QL_ERR_ARG, "eps must be >= 0, got %g", (double)eps);
  if (M == 0) return ok();
  if (!x || !shift || !scale || !out || (out_kind != QL_OPERAND_PLAIN && !row_scale))
    return fail(QL_ERR_ARG, "null x / shift / scale / out / row_scale pointer");
  if (!aligned16(x) || !aligned16(shift) || !aligned16(scale) ||
      (out_kind == QL_OPERAND_I8_PER_TOKEN ? ((uintptr_t)out & 7) != 0 : !aligned16(out)))
    return fail(QL_ERR_ALIGN, "x, shift, scale and out must be 16-byte aligned (int8 out: 8-byte)");
  const int kind = out_kind == QL_OPERAND_PLAIN ? kOperandPlain : out_kind == QL_OPERAND_I8_PER_TOKEN ? kOperandI8 : kOperandF16;
  const hipError_t e = adaln_launch(kind, x_dtype, mod_dtype, x, shift, scale, out, row_scale, M, K, eps,
                                    (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "adaln_modulate launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_adaln_modulate_f16(int x_dtype, const void* x, int mod_dtype, const void* shift, const void* scale,
                               void* x16, float* row_scale, int64_t M, int64_t K, float eps, void* stream) {
  return qlinear_adaln_modulate(QL_OPERAND_F16_ROWSCALED, x_dtype, x, mod_dtype, shift, scale, x16, row_scale, M, K, eps,
                                stream);
}

int qlinear_qk_norm_rope(int dtype, const void* qkv, const void* q_norm, const void* k_norm, const float* cos_t,
                         const float* sin_t, void* q, void* k, void* v, int64_t L, int64_t H, int64_t D,
                         int64_t L_out, int64_t l_offset, float eps, void* stream) {
  if (dtype != QL_F16 && dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "dtype %s (%d) unsupported, expected float16/bfloat16", dtype_name(dtype), dtype);
  if (D != 128) return fail(QL_ERR_SHAPE, "head dim must be 128, got %lld", (long long)D);
  if (L < 0 || H <= 0 || l_offset < 0 || L_out < 0 || l_offset + L > L_out || L_out > (1 << 24) ||
      H > 4096 || L * H > ((int64_t)1 << 31))
    return fail(QL_ERR_SHAPE, "expected qkv [L, 3, H, 128] written to rows [l_offset, l_offset + L) of [H, L_out, 128]; "
                "got L=%lld H=%lld L_out=%lld l_offset=%lld", (long long)L, (long long)H, (long long)L_out,
                (long long)l_offset);
  if (!(eps >= 0.0f)) return fail(QL_ERR_ARG, "eps must be >= 0, got %g", (double)eps);
  if (L == 0) return ok();
  if (!qkv || !q_norm || !k_norm || !cos_t || !sin_t || !q || !k || !v)
    return fail(QL_ERR_ARG, "null qkv / q_norm / k_norm / cos / sin / q / k / v pointer");
  const void* ptrs[] = {qkv, q_norm, k_norm, cos_t, sin_t, q, k, v};
  for (const void* p : ptrs)
    if ((uintptr_t)p & 3u) return fail(QL_ERR_ALIGN, "every pointer must be 4-byte aligned (%p)", p);
  const hipError_t e = qk_norm_rope_launch(dtype, qkv, q_norm, k_norm, cos_t, sin_t, q, k, v, L, H, L_out, l_offset,
                                           eps, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "qk_norm_rope launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_stream_read(const void* buf, int64_t bytes, uint32_t* out, void* stream) {
  if (bytes < 16 || bytes % 16 != 0) return fail(QL_ERR_SHAPE, "bytes must be a positive multiple of 16, got %lld",
                                                 (long long)bytes);
  if (!buf || !out) return fail(QL_ERR_ARG, "null buf / out pointer");
  if (!aligned16(buf)) return fail(QL_ERR_ALIGN, "buf must be 16-byte aligned");
  int cus = 0;
  if (int rc = device_cus(-1, &cus)) return rc;
  const hipError_t e = stream_read_launch(buf, bytes, out, cus, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "stream_read launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_gated_residual(int dtype, void* out, const void* x, const void* gate, const void* y, int64_t M, int64_t K,
                           void* stream) {
  if (dtype != QL_F32 && dtype != QL_F16 && dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "dtype %s (%d) unsupported, expected float32/float16/bfloat16", dtype_name(dtype), dtype);
  if (M < 0 || K <= 0 || K % 8 != 0 || K > INT32_MAX || M > INT64_MAX / 8 / K)
    return fail(QL_ERR_SHAPE, "x must be [M, K] with K %% 8 == 0, got [%lld, %lld]", (long long)M, (long long)K);
  if (M == 0) return ok();
  if (!out || !x || !gate || !y) return fail(QL_ERR_ARG, "null out / x / gate / y pointer");
  if (!aligned16(out) || !aligned16(x) || !aligned16(gate) || !aligned16(y))
    return fail(QL_ERR_ALIGN, "out, x, gate and y must be 16-byte aligned");
  const hipError_t e = gated_residual_launch(dtype, out, x, gate, y, M, K, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "gated_residual launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_w4a4_auto_splits(int64_t M, int64_t N, int64_t K, int device) {
  if (M < 0 || N <= 0 || K < 32 || K % 32 != 0 || M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > (1 << 30)) {
    fail(QL_ERR_SHAPE, "expected M >= 0, N > 0, K %% 32 == 0, K >= 32; got M=%lld N=%lld K=%lld", (long long)M,
         (long long)N, (long long)K);
    return -QL_ERR_SHAPE;
  }
  int cus = 0;
  if (int rc = device_cus(device, &cus)) return -rc;
  return w4a4_reference_splits(M, N, K, cus);
}

size_t qlinear_w4a4_workspace_bytes(int64_t M, int64_t N, int64_t K, int splits, int device) {
  if (M <= 0 || N <= 0 || K < 32 || K % 32 != 0 || splits < 0 || splits > kW4A4MaxSplits) return 0;
  int cus = 0;
  if (splits == 0 && device_cus(device, &cus) != QL_OK) return 0;
  const int s = splits == 0 ? w4a4_reference_splits(M, N, K, cus) : splits;
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * sizeof(float) : 0;
}

int qlinear_w4a4_gemm(int out_dtype, const void* a_q4, const float* a_scale, const void* b_q4, const float* b_scale,
                      const void* bias, void* y, int64_t M, int64_t N, int64_t K, int qblock, int splits,
                      void* workspace, size_t workspace_bytes, void* stream) {
  if (out_dtype != QL_F32 && out_dtype != QL_F16 && out_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "out dtype %s (%d) unsupported, expected float32/float16/bfloat16", dtype_name(out_dtype),
                out_dtype);
  if (qblock != 32 && qblock != 16) return fail(QL_ERR_ARG, "qblock must be 32 or 16, got %d", qblock);
  if (M < 0 || N <= 0 || K < 32 || K % 32 != 0 || M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > (1 << 30))
    return fail(QL_ERR_SHAPE, "expected A [M, K/2], B [N, K/2] with K %% 32 == 0, K >= 32, N > 0; got M=%lld N=%lld "
                "K=%lld", (long long)M, (long long)N, (long long)K);
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
  if (tiles > INT32_MAX) return fail(QL_ERR_SHAPE, "too many 128 x 128 tiles (M=%lld N=%lld)", (long long)M, (long long)N);
  if (splits < 0 || splits > kW4A4MaxSplits)
    return fail(QL_ERR_ARG, "splits must be in [0, %d], got %d", kW4A4MaxSplits, splits);
  if (M == 0) return ok();
  if (!a_q4 || !a_scale || !b_q4 || !b_scale || !y) return fail(QL_ERR_ARG, "null a_q4 / a_scale / b_q4 / b_scale / y pointer");
  if (splits == 0) {
    int cus = 0;
    if (int rc = device_cus(-1, &cus)) return rc;
    splits = w4a4_reference_splits(M, N, K, cus);
  }
  const size_t need = splits > 1 ? (size_t)splits * (size_t)M * (size_t)N * sizeof(float) : 0;
  if (need && (!workspace || workspace_bytes < need))
    return fail(QL_ERR_WORKSPACE, "split-K over %d splits needs a workspace of %zu bytes (fp32 [%d, %lld, %lld]), got "
                "%zu at %p", splits, need, splits, (long long)M, (long long)N, workspace_bytes, workspace);
  if (need && ((uintptr_t)workspace & 3u)) return fail(QL_ERR_ALIGN, "workspace must be 4-byte aligned");
  if (!aligned16(a_q4) || !aligned16(b_q4)) return fail(QL_ERR_ALIGN, "a_q4 and b_q4 must be 16-byte aligned");
  if (((uintptr_t)a_scale & 3u) || ((uintptr_t)b_scale & 3u))
    return fail(QL_ERR_ALIGN, "a_scale and b_scale must be 4-byte aligned");
  W4A4Params p{};
  p.a = a_q4;
  p.as = a_scale;
  p.b = b_q4;
  p.bs = b_scale;
  p.bias = bias;
  p.y = y;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.out_dtype = out_dtype;
  p.tiles_m = (int)((M + 127) / 128);
  p.tiles_n = (int)((N + 127) / 128);
  // the reference's k-tiles of 4 blocks of 32 K (128 K) are this kernel's int4 stages
  const int k_tiles = (int)((K / 32 + 3) / 4);
  p.splits = splits;
  p.stages_per_split = (k_tiles + splits - 1) / splits;
  p.partial = (float*)workspace;
  const hipError_t e = w4a4_launch(qblock, p, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "w4a4 launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_rotate_rows_to_f16(int x_dtype, const void* x, const float* signs, int group, void* x16, float* row_scale,
                               int64_t M, int64_t K, void* stream) {
  if (x_dtype != QL_F32 && x_dtype != QL_F16 && x_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "x dtype %s (%d) unsupported, expected float32/float16/bfloat16", dtype_name(x_dtype),
                x_dtype);
  if (group != 32 && group != 64 && group != 128)
    return fail(QL_ERR_ARG, "rotation group must be 32, 64 or 128, got %d", group);
  if (M < 0 || M > INT32_MAX || K <= 0 || K % group != 0 || K > 16384)
    return fail(QL_ERR_SHAPE, "x must be [M, K] with K %% %d == 0 and K <= 16384, got [%lld, %lld]", group,
                (long long)M, (long long)K);
  if (M == 0) return ok();
  if (!x || !signs || !x16 || !row_scale) return fail(QL_ERR_ARG, "null x / signs / x16 / row_scale pointer");
  if (!aligned16(x) || !aligned16(x16)) return fail(QL_ERR_ALIGN, "x and x16 must be 16-byte aligned");
  if ((uintptr_t)signs & 3u) return fail(QL_ERR_ALIGN, "signs must be 4-byte aligned");
  const hipError_t e = rotate_rows_to_f16_launch(x_dtype, group, x, signs, x16, row_scale, M, K, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "rotate_rows_to_f16 launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_heads_gather(int out_kind, int dtype, const void* o, int64_t H, int64_t L_all, int64_t D, int64_t l_offset,
                         int64_t rows, const void* extra, int64_t E, void* out, float* row_scale, void* stream) {
  if (out_kind != QL_OPERAND_F16_ROWSCALED && out_kind != QL_OPERAND_PLAIN && out_kind != QL_OPERAND_I8_PER_TOKEN)
    return fail(QL_ERR_ARG, "out_kind must be QL_OPERAND_F16_ROWSCALED, QL_OPERAND_PLAIN or QL_OPERAND_I8_PER_TOKEN, got %d",
                out_kind);
  if (dtype != QL_F16 && dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "dtype %s (%d) unsupported, expected float16/bfloat16", dtype_name(dtype), dtype);
  if (D != 128) return fail(QL_ERR_SHAPE, "head dim must be 128, got %lld", (long long)D);
  if (H <= 0 || rows < 0 || l_offset < 0 || l_offset + rows > L_all || L_all > INT32_MAX || E < 0 || E % 8 != 0 ||
      H * 128 + E > 16384)
    return fail(QL_ERR_SHAPE, "expected o [H, L_all, 128] rows [l_offset, l_offset + rows) and extra [rows, E] with "
                "E %% 8 == 0, H * 128 + E <= 16384; got H=%lld L_all=%lld l_offset=%lld rows=%lld E=%lld", (long long)H,
                (long long)L_all, (long long)l_offset, (long long)rows, (long long)E);
  if (rows == 0) return ok();
  if (!o || !out || (out_kind != QL_OPERAND_PLAIN && !row_scale) || (E > 0 && !extra))
    return fail(QL_ERR_ARG, "null o / extra / out / row_scale pointer");
  if (!aligned16(o) || (E > 0 && !aligned16(extra)) ||
      (out_kind == QL_OPERAND_I8_PER_TOKEN ? ((uintptr_t)out & 7) != 0 : !aligned16(out)))
    return fail(QL_ERR_ALIGN, "o, extra and out must be 16-byte aligned (int8 out: 8-byte)");
  const int kind = out_kind == QL_OPERAND_PLAIN ? kOperandPlain : out_kind == QL_OPERAND_I8_PER_TOKEN ? kOperandI8 : kOperandF16;
  const hipError_t e = heads_gather_launch(kind, dtype, o, H, L_all, l_offset, rows, E > 0 ? extra : nullptr, E, out,
                                           row_scale, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "heads_gather launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_heads_to_f16(int dtype, const void* o, int64_t H, int64_t L_all, int64_t D, int64_t l_offset, int64_t rows,
                         const void* extra, int64_t E, void* x16, float* row_scale, void* stream) {
  return qlinear_heads_gather(QL_OPERAND_F16_ROWSCALED, dtype, o, H, L_all, D, l_offset, rows, extra, E, x16, row_scale,
                              stream);
}

int qlinear_quantize_int8_block32(int x_dtype, const void* x, int8_t* q, float* scale, int64_t rows, int64_t K,
                                  void* stream) {
  if (x_dtype != QL_F32 && x_dtype != QL_F16 && x_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "unsupported dtype %s (%d), expected float32/float16/bfloat16", dtype_name(x_dtype),
                x_dtype);
  if (rows < 0 || K < 32 || K % 32 != 0 || rows * (K / 32) > ((int64_t)1 << 40))
    return fail(QL_ERR_SHAPE, "x must be [rows, K] with K %% 32 == 0, got [%lld, %lld]", (long long)rows, (long long)K);
  if (rows == 0) return ok();
  if (!x || !q || !scale) return fail(QL_ERR_ARG, "null x / q / scale pointer");
  if (!aligned16(x) || !aligned16(q) || ((uintptr_t)scale & 3u))
    return fail(QL_ERR_ALIGN, "x and q must be 16-byte aligned, scale 4-byte aligned");
  const hipError_t e = quantize_int8_block32_launch(x_dtype, x, q, scale, rows * (K / 32), (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "quantize_int8_block32 launch failed: %s", hipGetErrorString(e));
  return ok();
}

int qlinear_gemm_int8_block32(int out_dtype, const int8_t* a, const float* a_scale, const int8_t* b, const float* b_scale,
                              const void* bias, void* y, int64_t M, int64_t N, int64_t K, void* stream) {
  if (out_dtype != QL_F32 && out_dtype != QL_F16 && out_dtype != QL_BF16)
    return fail(QL_ERR_DTYPE, "out dtype %s (%d) unsupported, expected float32/float16/bfloat16", dtype_name(out_dtype),
                out_dtype);
  if (M < 0 || N <= 0 || K < 32 || K % 32 != 0 || M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > (1 << 30))
    return fail(QL_ERR_SHAPE, "expected A [M, K], B [N, K] with K %% 32 == 0, K >= 32, N > 0; got M=%lld N=%lld K=%lld",
                (long long)M, (long long)N, (long long)K);
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
  if (tiles > INT32_MAX) return fail(QL_ERR_SHAPE, "too many 128 x 128 tiles (M=%lld N=%lld)", (long long)M, (long long)N);
  if (M == 0) return ok();
  if (!a || !a_scale || !b || !b_scale || !y) return fail(QL_ERR_ARG, "null a / a_scale / b / b_scale / y pointer");
  if (!aligned16(a) || !aligned16(b)) return fail(QL_ERR_ALIGN, "a and b must be 16-byte aligned");
  if (((uintptr_t)a_scale & 3u) || ((uintptr_t)b_scale & 3u))
    return fail(QL_ERR_ALIGN, "a_scale and b_scale must be 4-byte aligned");
  W4A4Params p{};
  p.a = a;
  p.as = a_scale;
  p.b = b;
  p.bs = b_scale;
  p.bias = bias;
  p.y = y;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.out_dtype = out_dtype;
  p.tiles_m = (int)((M + 127) / 128);
  p.tiles_n = (int)((N + 127) / 128);
  const hipError_t e = int8_block32_launch(p, (hipStream_t)stream);
  if (e != hipSuccess) return fail(QL_ERR_LAUNCH, "gemm_int8_block32 launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"
