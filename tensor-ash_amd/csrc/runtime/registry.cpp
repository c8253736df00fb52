// KERNEL_SPECS registry, ML_KERNEL parsing, shape routing, split-K and
// GEMV geometry, and the pure helpers of the measured tuner.
#include <algorithm>
#include <cctype>
#include <cstdlib>
#include <sstream>

#include "internal.hpp"

namespace tensor_ash {

// Data-driven registry (role of src/pipeline/catalog.rs:129-376): one
// declaration per gfx950 kernel; the ML_KERNEL names and the routing all
// derive from it.  `symbol` is the code-object symbol stem: GEMM entries
// add "_vec" / "_gen" (aligned / ragged loads), GEMV entries add "_m1",
// "_m2", "_m4", "_m8" (rows per launch) and "_dual" (SwiGLU pair).
const KernelSpec KERNEL_SPECS[] = {
    {"f32_m256n256", 256, 256, 32, KernelKind::GemmF32, "ta_gemm_f32_m256n256", "large"},
    {"f32_m256n128", 256, 128, 16, KernelKind::GemmF32, "ta_gemm_f32_m256n128", ""},
    {"f32_m128n128", 128, 128, 16, KernelKind::GemmF32, "ta_gemm_f32_m128n128", "medium"},
    {"f32_m128n64", 128, 64, 16, KernelKind::GemmF32, "ta_gemm_f32_m128n64", ""},
    {"f32_m64n64", 64, 64, 16, KernelKind::GemmF32, "ta_gemm_f32_m64n64", "small"},
    {"f32_m64n256", 64, 256, 16, KernelKind::GemmF32, "ta_gemm_f32_m64n256", ""},
    {"f32_m32n128", 32, 128, 16, KernelKind::GemmF32, "ta_gemm_f32_m32n128", ""},
    {"f32_m32n64", 32, 64, 16, KernelKind::GemmF32, "ta_gemm_f32_m32n64", ""},
    {"f16w_m256n256", 256, 256, 32, KernelKind::GemmF16w, "ta_gemm_f16w_m256n256", ""},
    {"f16w_m256n128", 256, 128, 16, KernelKind::GemmF16w, "ta_gemm_f16w_m256n128", ""},
    {"f16w_m128n128", 128, 128, 16, KernelKind::GemmF16w, "ta_gemm_f16w_m128n128", ""},
    {"f16w_m128n64", 128, 64, 16, KernelKind::GemmF16w, "ta_gemm_f16w_m128n64", ""},
    {"f16w_m64n64", 64, 64, 16, KernelKind::GemmF16w, "ta_gemm_f16w_m64n64", ""},
    {"f16w_mfma_m256n256", 256, 256, 64, KernelKind::GemmF16Mfma, "ta_gemm_h16_m256n256", ""},
    {"f16w_mfma_m128n128", 128, 128, 64, KernelKind::GemmF16Mfma, "ta_gemm_h16_m128n128",
     "f16w_coopmat_aligned"},
    {"f16w_mfma_m128n64", 128, 64, 64, KernelKind::GemmF16Mfma, "ta_gemm_h16_m128n64",
     "f16w_coopmat_m128n64"},
    {"f16w_mfma_m64n128", 64, 128, 64, KernelKind::GemmF16Mfma, "ta_gemm_h16_m64n128",
     "f16w_coopmat_m64n128"},
    {"f16w_mfma_m64n64", 64, 64, 64, KernelKind::GemmF16Mfma, "ta_gemm_h16_m64n64",
     "f16w_coopmat_m64n64"},
    {"f16w_sk_m128n128", 128, 128, 64, KernelKind::GemmF16Sk, "ta_gemm_h16sk_m128n128", ""},
    {"f16w_sk_m128n64", 128, 64, 64, KernelKind::GemmF16Sk, "ta_gemm_h16sk_m128n64", ""},
    {"f16w_sk_m64n128", 64, 128, 64, KernelKind::GemmF16Sk, "ta_gemm_h16sk_m64n128", ""},
    {"f16w_a16_m256n256", 256, 256, 64, KernelKind::GemmA16, "ta_gemm_a16_m256n256", ""},
    {"f16w_a16_m128n128", 128, 128, 64, KernelKind::GemmA16, "ta_gemm_a16_m128n128",
     "f16w_a16_coopmat_aligned"},
    {"f16w_a16_m128n64", 128, 64, 64, KernelKind::GemmA16, "ta_gemm_a16_m128n64",
     "f16w_a16_coopmat_m128n64"},
    {"f16w_a16_m64n128", 64, 128, 64, KernelKind::GemmA16, "ta_gemm_a16_m64n128",
     "f16w_a16_coopmat_m64n128"},
    {"f16w_a16_m64n64", 64, 64, 64, KernelKind::GemmA16, "ta_gemm_a16_m64n64",
     "f16w_a16_coopmat_m64n64"},
    {"f16w_gemv_packed_t64", 8, 64, 0, KernelKind::GemvF16Packed, "ta_gemv_f16_t64",
     "f16w_row_packed"},
    {"f16w_gemv_packed_t32", 8, 32, 0, KernelKind::GemvF16Packed, "ta_gemv_f16_t32", ""},
    {"f16w_gemv_row", 8, 64, 0, KernelKind::GemvF16Row, "ta_gemv_f16_t64", "f16w_row"},
    {"f32_gemv_row", 8, 64, 0, KernelKind::GemvF32Row, "ta_gemv_f32_t64", "row_bda,row"},
};
const size_t KERNEL_SPECS_LEN = sizeof(KERNEL_SPECS) / sizeof(KERNEL_SPECS[0]);

size_t registry_index(const char *name) {
  for (size_t i = 0; i < KERNEL_SPECS_LEN; ++i)
    if (std::string(KERNEL_SPECS[i].name) == name)
      return i;
  fail(std::string("no kernel named ") + name);
}

namespace {
std::string trim_lower(const std::string &v) {
  size_t b = 0, e = v.size();
  while (b < e && std::isspace((unsigned char)v[b]))
    ++b;
  while (e > b && std::isspace((unsigned char)v[e - 1]))
    --e;
  std::string s = v.substr(b, e - b);
  for (auto &c : s)
    c = (char)std::tolower((unsigned char)c);
  return s;
}
} // namespace

// src/pipeline/catalog.rs:162-180: case-insensitive, surrounding
// whitespace ignored, "" and "auto" mean Auto.
KernelSelection KernelSelection::parse(const std::string &value) {
  const std::string v = trim_lower(value);
  if (v.empty() || v == "auto")
    return KernelSelection{};
  for (size_t i = 0; i < KERNEL_SPECS_LEN; ++i) {
    if (v == KERNEL_SPECS[i].name)
      return KernelSelection{i};
    std::stringstream aliases(KERNEL_SPECS[i].aliases);
    std::string a;
    while (std::getline(aliases, a, ','))
      if (!a.empty() && v == a)
        return KernelSelection{i};
  }
  std::string names;
  for (size_t i = 0; i < KERNEL_SPECS_LEN; ++i)
    names += std::string(", ") + KERNEL_SPECS[i].name;
  fail("invalid ML_KERNEL '" + v + "', expected one of auto" + names);
}

KernelSelection KernelSelection::from_env() {
  const char *v = std::getenv("ML_KERNEL");
  return parse(v ? v : "auto");
}

namespace {
uint32_t div_ceil(uint32_t a, uint32_t b) { return (a + b - 1) / b; }
} // namespace

// Shapes the pipelined f16-MFMA kernels (`_lds` code objects) take: whole
// 64-deep K stages and 16-byte B rows.
bool gemm_lds_ok(const ResolvedMatmul &d) { return d.k > 0 && d.k % 64 == 0 && d.n % 8 == 0; }
// Pipelined f16w tiles that also have a dual (SwiGLU pair) kernel,
// ta_gemm_h16dual_<tile>_lds.
bool f16_dual_tile(const KernelSpec &s) {
  return s.kind == KernelKind::GemmF16Mfma &&
         ((s.tile_m == 128 && (s.tile_n == 128 || s.tile_n == 64)) ||
          (s.tile_m == 64 && (s.tile_n == 128 || s.tile_n == 64)));
}

// Threads of the _mi16 kernel of a tile height (32: 128, else 256).
uint32_t mi16_threads(uint32_t tile_m) { return tile_m == 32 ? 128u : 256u; }

// The ta_gemm_f32_<tile>_mi16 kernels (256x256, and the split-K stage-1
// tiles 64x256 and 32x128) take whole tiles of f32 A and B and walk each
// K window ta_mi16_stages(tile_m) 16-deep stages at a time; `planes` K
// windows of equal length holding whole loops (the split window rule gives
// that when K is a multiple of 16 * stages * planes); 32-bit per-lane load
// offsets span a tile's A rows and 16 rows of B.
bool f32_mi16_ok(const ResolvedMatmul &d, uint32_t tile_m, uint32_t tile_n, uint32_t planes) {
  // 64 x 64 only as split-K stage 1 (plain GEMMs keep their measured routes)
  const bool tile = (tile_m == 256 && tile_n == 256) || (tile_m == 64 && tile_n == 256) ||
                    (tile_m == 32 && tile_n == 128) ||
                    (((tile_m == 64 && tile_n == 64) || (tile_m == 32 && tile_n == 64)) && planes > 1);
  const uint64_t loop = 16ull * ta_mi16_stages((int)tile_m, (int)tile_n);
  return tile && planes >= 1 && !d.a_f16 && !d.b_f16 && d.m % tile_m == 0 && d.n % tile_n == 0 &&
         d.k > 0 && d.k % (loop * planes) == 0 && (uint64_t)tile_m * d.k * 4 < (1ull << 32) &&
         16ull * d.n * 4 < (1ull << 32);
}

bool kernel_supports(const KernelSpec &s, const ResolvedMatmul &d) {
  // The 256x256 f16-MFMA tiles exist only as pipelined kernels.
  if ((s.kind == KernelKind::GemmF16Mfma || s.kind == KernelKind::GemmA16) && s.tile_m == 256 &&
      !gemm_lds_ok(d))
    return false;
  if (d.a_f16)
    return s.kind == KernelKind::GemmA16;
  if (d.packed_b)
    return s.kind == KernelKind::GemvF16Packed && d.m <= kGemvMaxRows && d.batch == 1 &&
           d.n % s.tile_n == 0;
  switch (s.kind) {
  case KernelKind::GemmF32:
    return !d.b_f16;
  case KernelKind::GemmF16w:
  case KernelKind::GemmF16Mfma:
    return d.b_f16;
  case KernelKind::GemmA16:
    return false;
  case KernelKind::GemmF16Sk:
    return d.b_f16 && !d.a_f16 && gemm_lds_ok(d);
  case KernelKind::GemvF16Row:
    return d.b_f16 && d.batch == 1 && d.m <= kGemvMaxRows && d.n % 4 == 0;
  case KernelKind::GemvF32Row:
    return !d.b_f16 && d.batch == 1 && d.m <= kGemvMaxRows && d.n % 2 == 0;
  case KernelKind::GemvF16Packed:
    return false;
  }
  return false;
}

// Largest tile of `names` whose grid covers every CU once, else the last.
static size_t pick_tile(const char *const *names, int count, uint32_t cus, uint32_t batch,
                        uint32_t m, uint32_t n) {
  for (int i = 0; i < count; ++i) {
    const KernelSpec &s = KERNEL_SPECS[registry_index(names[i])];
    const uint64_t tiles = (uint64_t)batch * div_ceil(m, s.tile_m) * div_ceil(n, s.tile_n);
    if (tiles >= cus)
      return registry_index(names[i]);
  }
  return registry_index(names[count - 1]);
}

// f16-MFMA tile.  Pipelined shapes: 256x256 when that grid covers every
// CU; else the largest of 128x128 and 128x64 (8 waves) whose grid still
// covers 60% of the CUs; else, for f16 weights with deep K (>= 64 stages)
// whose 128x64 grid fits the CUs twice over, the split-K kernel; else
// 64x64 (4 waves).  Measured on the M = 512 prefill shapes (a K step of
// these kernels costs latency, so a tile's time follows its K steps: small
// tiles win while the grid is small, and a deep K is best split).  Other
// shapes take the largest register-staged tile covering every CU.
static size_t pick_f16_mfma(bool a16, uint32_t cus, uint32_t batch, uint32_t m, uint32_t n,
                            uint32_t k) {
  static const char *mfma16_tiles[] = {"f16w_mfma_m128n128", "f16w_mfma_m128n64",
                                       "f16w_mfma_m64n128", "f16w_mfma_m64n64"};
  static const char *a16_tiles[] = {"f16w_a16_m128n128", "f16w_a16_m128n64",
                                    "f16w_a16_m64n128", "f16w_a16_m64n64"};
  ResolvedMatmul d;
  d.m = m;
  d.n = n;
  d.k = k;
  if (!gemm_lds_ok(d))
    return pick_tile(a16 ? a16_tiles : mfma16_tiles, 4, cus, batch, m, n);
  const std::string pre = a16 ? "f16w_a16_" : "f16w_mfma_";
  auto tiles = [&](uint32_t bm, uint32_t bn) {
    return (uint64_t)batch * div_ceil(m, bm) * div_ceil(n, bn);
  };
  // Chosen with the weights streamed from HBM (a model's layers together
  // exceed the last-level cache): with more columns than rows, 64 x 128
  // tiles beat 128 x 64 at the same tile count (512x2560x2048: 17.9 against
  // 19.3 us), and deep-K shapes split 128 x 128 tiles rather than 128 x 64
  // (512x2048x5632: 26.4 us with 4 splits against 29.5 with 2).
  const uint64_t most = cus * 6ull / 10;
  const bool wide = n > m && tiles(64, 128) == tiles(128, 64);
  const char *tile = tiles(256, 256) >= cus   ? "m256n256"
                     : tiles(128, 128) >= most ? "m128n128"
                     : tiles(128, 64) >= most  ? (wide ? "m64n128" : "m128n64")
                                               : "m64n64";
  if (!a16 && std::string(tile) == "m64n64" && k / 64 >= 64 && 2 * tiles(128, 64) <= cus)
    return registry_index(2 * tiles(128, 128) <= cus ? "f16w_sk_m128n128" : "f16w_sk_m128n64");
  return registry_index((pre + tile).c_str());
}

// Shape heuristic for 256-CU MI355X (role of src/pipeline/mod.rs:293-360
// and selection.rs:89-172; the reference's NVIDIA-tuned tables are not a
// target): decode shapes (M <= 8, one batch) stream the weights through
// the GEMV; f16 weights with M, N >= 64 run on the f16 MFMA (A rounded to
// f16 RNE, like the reference's coopmat route), smaller f16-weight
// shapes widen B exactly on the FP32 MFMA; f16 activations take the a16
// kernels.  FP32 tiles: the largest whose grid still covers every CU once.
size_t heuristic_kernel_index(uint32_t cus, uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                              bool b_f16, bool packed_b, bool a_f16) {
  static const char *f32_tiles[] = {"f32_m256n256", "f32_m256n128", "f32_m128n128",
                                    "f32_m128n64", "f32_m64n64"};
  static const char *f16w_tiles[] = {"f16w_m256n256", "f16w_m256n128", "f16w_m128n128",
                                     "f16w_m128n64", "f16w_m64n64"};
  if (a_f16)
    return pick_f16_mfma(true, cus, batch, m, n, k);
  if (packed_b)
    return registry_index(n % 64 == 0 ? "f16w_gemv_packed_t64" : "f16w_gemv_packed_t32");
  if (batch == 1 && m <= kGemvMaxRows && n % (b_f16 ? 4 : 2) == 0)
    return registry_index(b_f16 ? "f16w_gemv_row" : "f32_gemv_row");
  if (b_f16 && m >= 64 && n >= 64)
    return pick_f16_mfma(false, cus, batch, m, n, k);
  return pick_tile(b_f16 ? f16w_tiles : f32_tiles, 5, cus, batch, m, n);
}

// Every kernel that can run the shape (role of pipeline/mod.rs:491-535).
std::vector<size_t> tune_candidate_indices(const ResolvedMatmul &dims) {
  std::vector<size_t> out;
  for (size_t i = 0; i < KERNEL_SPECS_LEN; ++i)
    if (kernel_supports(KERNEL_SPECS[i], dims))
      out.push_back(i);
  return out;
}

// ---- split-K (src/executor/splitk2.rs:36-271, retuned for 256 CUs) ----

// Skinny split-K shapes take 64-column tiles (64 x 64, or 32 x 64 for
// outputs of at most 32 rows): at the same workgroup count their K windows
// are longer than those of a tile spanning N, so the partial planes the
// reduce reads are fewer (the tiles of one window share its A rows in one
// XCD's L2).  Measured, stage 1 + reduce: 64 x 256 x 65536 32.8 us against
// 36.8 us with 64 x 256 tiles; 32 x 128 x 131072 30.4 against 31.8 us
// with 32 x 128 tiles.
// Outputs of at least 128 x 128 whose sides are whole 64-column tiles and
// whose K splits into windows of whole eight-stage loops at up to 16
// planes (K % 2048 == 0) take the pipelined 64 x 64 tile as well: a
// 256 x 256 x 16384 op then runs 16 tiles x 16 windows of 1024 on the
// FP32-MFMA pipeline (38.7-39.8 us on the 128 x 128 register-staged tile
// at 64 planes).
const KernelSpec &splitk_stage1_spec(uint32_t m, uint32_t n, uint32_t k) {
  const bool pipelined64 = m % 64 == 0 && n % 64 == 0 && k % 2048 == 0;
  const char *name = m >= 128 && n >= 128 && !pipelined64 ? "f32_m128n128"
                     : m <= 32                            ? "f32_m32n64"
                                                          : "f32_m64n64";
  return KERNEL_SPECS[registry_index(name)];
}

// K splits per output tile of the ta_gemm_h16sk_* kernels (one workgroup
// per CU at a time, LDS-bound): the count in 1..8 (at least 4 K stages
// per split) minimising rounds x stages per split, where a round is one
// pass of workgroups over the CUs; ties go to fewer splits (less partial
// traffic).  TA_H16_SPLITS fixes the count (route control for
// measurements).
uint32_t h16sk_splits(uint32_t cus, uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                      uint32_t tile_m, uint32_t tile_n) {
  const uint64_t tiles = (uint64_t)batch * div_ceil(m, tile_m) * div_ceil(n, tile_n);
  const uint32_t steps = std::max(1u, k / 64);
  if (const char *env = std::getenv("TA_H16_SPLITS"))
    return std::clamp<uint32_t>((uint32_t)std::strtoul(env, nullptr, 10), 1u, std::min(steps, 64u));
  uint32_t best = 1;
  uint64_t best_cost = UINT64_MAX;
  for (uint32_t s = 1; s <= 8 && s <= steps; ++s) {
    if (s > 1 && steps / s < 4)
      break;
    const uint64_t rounds = (tiles * s + cus - 1) / cus;
    const uint64_t cost = rounds * ((steps + s - 1) / s);
    if (cost < best_cost) {
      best_cost = cost;
      best = s;
    }
  }
  return best;
}

uint32_t gemm_threads(const KernelSpec &s) {
  if (s.tile_m == 256 && s.tile_n == 256)
    return 512;
  return s.tile_m == 32 ? 128 : 256;
}

// Sub-windows per split for stage 1.  A stage-1 workgroup of the plain
// FP32 kernels keeps about one 16-deep K slab of A and B in flight, so HBM
// needs several hundred of them: aim for 4 workgroups per CU (8 for
// 128-thread tiles), with >= 256 K values per window.  The pipelined
// kernels (f32 operands, whole tiles, 64-aligned windows) keep three
// slabs in flight and are fastest at one workgroup per CU, which also
// halves the partial planes the reduce reads.  Always: grid z <= 65535,
// u32 scratch addressing and at most 256 MiB of partial planes.
uint32_t splitk_sub_splits(uint32_t cus, const ResolvedMatmul &d, uint32_t splits) {
  if (splits < 2 || d.batch == 0)
    return 1;
  const KernelSpec &s = splitk_stage1_spec(d.m, d.n, d.k);
  const uint64_t tiles = (uint64_t)d.batch * div_ceil(d.m, s.tile_m) * div_ceil(d.n, s.tile_n);
  const uint64_t plane = (uint64_t)d.batch * d.m * d.n;
  auto capped = [&](uint64_t t) {
    t = std::min<uint64_t>(t, 65535 / ((uint64_t)d.batch * splits));
    t = std::min<uint64_t>(t, std::max<uint64_t>(1, ((uint64_t)UINT32_MAX + 1) / (plane * splits)));
    t = std::min<uint64_t>(t, std::max<uint64_t>(1, (256ull << 20) / (plane * 4 * splits)));
    return (uint32_t)std::max<uint64_t>(1, t);
  };
  const uint32_t one_per_cu =
      capped(std::max<uint64_t>(1, (cus + tiles * splits - 1) / (tiles * splits)));
  if (f32_mi16_ok(d, s.tile_m, s.tile_n, splits * one_per_cu))
    return one_per_cu;
  const uint64_t target = (uint64_t)cus * (gemm_threads(s) <= 128 ? 8 : 4);
  uint64_t t = std::max<uint64_t>(1, (target + tiles * splits - 1) / (tiles * splits));
  t = std::min<uint64_t>(t, std::max<uint64_t>(1, d.k / ((uint64_t)splits * 256)));
  return capped(t);
}

// Plane groups per element for the split-K reduce: at least 8, then
// doubled (up to 256, keeping >= 4 planes per group) until quads * groups
// threads give every CU about two workgroups' worth of loads, so small
// outputs with many planes still spread over the chip.  A function of the shape
// only, which keeps the summation order fixed.
uint32_t splitk_reduce_groups(uint32_t cus, uint64_t quads, uint32_t planes) {
  uint32_t g = 8;
  while (g < 256 && 8ull * g <= planes && quads * g < 512ull * cus)
    g *= 2;
  while (g > 1 && g > planes)
    g /= 2;
  return g;
}

// Deep-K shapes whose data-parallel grid covers less than half of the CUs
// get enough K splits for ~2 workgroups per CU, keeping >= 256 K values
// per split so the partial planes never outweigh the MFMA work.
std::optional<uint32_t> heuristic_splits(uint32_t cus, uint32_t batch, uint32_t m, uint32_t n,
                                         uint32_t k) {
  if (batch == 0 || m <= 1 || n <= 1 || k < 1024)
    return std::nullopt;
  const KernelSpec &s = splitk_stage1_spec(m, n, k);
  const uint64_t tiles = (uint64_t)batch * div_ceil(m, s.tile_m) * div_ceil(n, s.tile_n);
  if (tiles * 2 >= cus)
    return std::nullopt;
  uint64_t wanted = (2ull * cus + tiles - 1) / tiles;
  // The pipelined stage-1 kernels (whole tiles, K windows of whole
  // pipeline loops) are fastest at one workgroup per CU: their windows
  // are then the longest and the partial planes fewest.
  const uint64_t one = std::max<uint64_t>(1, cus / tiles);
  if (m % s.tile_m == 0 && n % s.tile_n == 0 &&
      k % (16ull * ta_mi16_stages((int)s.tile_m, (int)s.tile_n) * one) == 0)
    wanted = one;
  const uint32_t max_splits = k / 256;
  for (uint32_t splits : {128u, 64u, 32u, 16u, 8u, 4u, 2u})
    if (splits <= wanted && splits <= max_splits)
      return splits;
  return std::nullopt;
}

// Split count for run_matmuls_split_k2(call, 0) (splitk2.rs:94-122): the
// heuristic when it applies, else enough splits for ~2 workgroups per CU
// with at least 32 K values each.
uint32_t default_num_k_splits(uint32_t cus, uint32_t batch, uint32_t m, uint32_t n, uint32_t k) {
  if (auto h = heuristic_splits(cus, batch, m, n, k))
    return *h;
  const KernelSpec &s = splitk_stage1_spec(m, n, k);
  const uint64_t tiles =
      (uint64_t)std::max(batch, 1u) * div_ceil(m, s.tile_m) * div_ceil(n, s.tile_n);
  if (tiles == 0)
    return 1;
  const uint64_t raw = std::max<uint64_t>(1, (2ull * cus + tiles - 1) / tiles);
  const uint64_t max_splits = std::max<uint64_t>(1, k / 32);
  return (uint32_t)std::min<uint64_t>({raw, max_splits, 0xFFFF});
}

// splitk2.rs:226-246.
void validate_scratch_geometry(uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                               uint32_t splits) {
  if (splits > k)
    fail("split-K2: splits=" + std::to_string(splits) + " exceeds K=" + std::to_string(k));
  unsigned __int128 e = (unsigned __int128)batch * m * n * splits;
  if (e > (unsigned __int128)UINT32_MAX + 1) {
    std::ostringstream o;
    o << "split-K2: batch*M*N*splits = " << (uint64_t)e << " exceeds u32 scratch addressing";
    fail(o.str());
  }
}

// splitk2.rs:155-188 (grid z limited to 65535 launches per batch*splits).
bool auto_route_fits(uint32_t batch, uint32_t m, uint32_t n, uint32_t k, uint32_t splits) {
  if (batch == 0 || m == 0 || n == 0 || splits < 2 || splits > 0xFFFF || splits > k)
    return false;
  const unsigned __int128 total = (unsigned __int128)batch * m * n;
  const unsigned __int128 elems = total * splits;
  if (elems > (unsigned __int128)UINT32_MAX + 1)
    return false;
  if (elems * 4 > kAutoScratchCapBytes)
    return false;
  return (uint64_t)batch * splits <= 65535;
}

// splitk2.rs:189-193: 16-byte aligned reservation inside the cap.
std::optional<uint64_t> checked_auto_scratch_end(uint64_t offset, uint64_t bytes) {
  if (bytes > UINT64_MAX - 15)
    return std::nullopt;
  const uint64_t rounded = (bytes + 15) / 16 * 16;
  if (offset > UINT64_MAX - rounded)
    return std::nullopt;
  const uint64_t end = offset + rounded;
  if (end > kAutoScratchCapBytes)
    return std::nullopt;
  return end;
}

// ---- GEMV geometry ----
// K granularity of a GEMV window: one unrolled load group of the kernel
// (4 waves x 64/(TW/CPL) rows x loads per group; CPL = 4 for f16, 2 for
// f32; 16 loads per group for 1-2 rows, 8 for 4-8 rows).
uint32_t gemv_unit(uint32_t tw, bool f32_weights, bool /*dual*/, uint32_t rows) {
  const uint32_t cpl = f32_weights ? 2 : 4;
  return 4 * (64 / (tw / cpl)) * (rows > 2 ? 8 : 16);
}

// ~3 workgroups per CU: K windows of at most 512 rows, a multiple of the
// kernel's unrolled group (host contract of the GEMV kernels).
GemvPlan plan_gemv(uint32_t cus, uint32_t rows, uint32_t n, uint32_t k, uint32_t tw, bool dual,
                   uint32_t unit) {
  GemvPlan p;
  p.tw = tw;
  p.mr = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
  p.tiles = div_ceil(n, tw);
  const uint32_t wanted = std::max(1u, div_ceil(3 * cus, p.tiles));
  uint32_t kchunk = div_ceil(k, wanted);
  // At one row, a grid of at least one tile per CU takes whole-K units:
  // no partials and no cross-workgroup reduction (32000 x 2048 lm_head:
  // 24.5 us against 26.7 with two windows of 1024; the smaller classes
  // measured slower with fewer, longer windows).
  if (p.mr == 1 && p.tiles >= cus)
    kchunk = k;
  if (const char *env = std::getenv("TA_GEMV_KCHUNK"))
    kchunk = (uint32_t)std::strtoul(env, nullptr, 10);
  kchunk = div_ceil(kchunk, unit) * unit;
  const uint32_t cap = 4096 / p.mr; // X-window rows the kernel stages in LDS
  kchunk = std::clamp(kchunk, unit, std::max(unit, cap / unit * unit));
  p.kchunk = kchunk;
  p.kchunks = div_ceil(k, kchunk);
  p.partial_bytes =
      p.kchunks > 1 ? (uint64_t)p.kchunks * p.tiles * (dual ? 2 : 1) * p.mr * tw * 4 : 0;
  return p;
}

std::vector<size_t> paired_conversion_picks(const std::vector<CvtCandidate> &ops) {
  std::vector<const void *> written;
  std::vector<size_t> picks;
  for (size_t i = 0; i < ops.size() && picks.size() < 2; ++i) {
    const CvtCandidate &c = ops[i];
    if (c.converts && std::find(written.begin(), written.end(), c.a_buffer) == written.end()) {
      const bool seen = !picks.empty() && ops[picks[0]].a_buffer == c.a_buffer &&
                        ops[picks[0]].a_ptr == c.a_ptr && ops[picks[0]].n == c.n;
      if (!seen)
        picks.push_back(i);
    }
    for (const void *w : c.writes)
      if (w)
        written.push_back(w);
  }
  if (picks.size() < 2)
    picks.clear();
  return picks;
}

// ---- tuner helpers (src/executor/tuning.rs:283-313) ----

std::optional<uint64_t> median(std::vector<uint64_t> s) {
  if (s.empty())
    return std::nullopt;
  std::sort(s.begin(), s.end());
  const size_t mid = s.size() / 2;
  if (s.size() % 2 == 0)
    return (uint64_t)(((unsigned __int128)s[mid - 1] + s[mid]) / 2);
  return s[mid];
}

// Interleaved candidate order: round 0 in registry order, then pairs of
// rounds walking forward and backward from a start that moves by half the
// list per pair, so every candidate sees every position equally often.
size_t candidate_at(size_t len, uint32_t round, size_t offset) {
  if (round == 0)
    return offset;
  const size_t pair = (round - 1) / 2;
  const size_t start = pair * ((len + 1) / 2) % len;
  if (round % 2 == 1)
    return (start + offset) % len;
  return (start + len - 1 - offset) % len;
}

bool TuneKey::operator<(const TuneKey &o) const {
  return std::tie(batch, m, n, k, b_f16) < std::tie(o.batch, o.m, o.n, o.k, o.b_f16);
}

// Persistent store (src/pipeline/tuning.rs:60-199): one header line that
// binds the HIP runtime version, the gfx arch and a hash of every loaded
// code object, then "B M N K kernel [splitk2=S] [bf16]" lines.
std::string tune_store_path(const Context &ctx) {
  std::string base;
  if (const char *x = std::getenv("XDG_CACHE_HOME"); x && *x)
    base = x;
  else if (const char *h = std::getenv("HOME"); h && *h)
    base = std::string(h) + "/.cache";
  else
    return "";
  std::string arch = ctx.arch();
  for (auto &c : arch)
    if (c == ':' || c == '/')
      c = '_';
  return base + "/tensor-ash/tuned_kernels_" + arch + ".txt";
}

std::string tune_header_line(const Context &ctx) {
  char hash[32];
  std::snprintf(hash, sizeof hash, "%016llx", (unsigned long long)ctx.code_object_hash());
  return "tensor-ash-tune-v3 hip=" + std::to_string(ctx.runtime_version()) +
         " arch=" + ctx.arch() + " kernels=" + hash;
}

std::map<TuneKey, TuneEntry> parse_tune_store(const std::string &text,
                                              const std::string &header) {
  std::map<TuneKey, TuneEntry> map;
  std::istringstream in(text);
  std::string line;
  if (!std::getline(in, line) || line != header)
    return map;
  while (std::getline(in, line)) {
    std::istringstream ls(line);
    long long b, m, n, k;
    std::string name;
    if (!(ls >> b >> m >> n >> k >> name))
      continue;
    if (b <= 0 || m <= 0 || n <= 0 || k <= 0 || b > UINT32_MAX || m > UINT32_MAX ||
        n > UINT32_MAX || k > UINT32_MAX)
      continue;
    size_t idx = KERNEL_SPECS_LEN;
    for (size_t i = 0; i < KERNEL_SPECS_LEN; ++i)
      if (name == KERNEL_SPECS[i].name)
        idx = i;
    if (idx == KERNEL_SPECS_LEN)
      continue;
    TuneEntry e{idx, std::nullopt};
    bool bf16 = false;
    std::string tok;
    while (ls >> tok) {
      if (tok.rfind("splitk2=", 0) == 0) {
        char *end = nullptr;
        const unsigned long s = std::strtoul(tok.c_str() + 8, &end, 10);
        if (end && *end == 0 && s >= 2 && s <= 0xFFFF)
          e.splitk2_splits = (uint32_t)s;
      } else if (tok == "bf16") {
        bf16 = true;
      }
    }
    map[TuneKey{(uint32_t)b, (uint32_t)m, (uint32_t)n, (uint32_t)k, bf16}] = e;
  }
  return map;
}

std::string format_tune_store(const std::map<TuneKey, TuneEntry> &map,
                              const std::string &header) {
  std::ostringstream o;
  o << header << "\n";
  for (const auto &[key, e] : map) {
    o << key.batch << " " << key.m << " " << key.n << " " << key.k << " "
      << KERNEL_SPECS[e.kernel].name;
    if (e.splitk2_splits)
      o << " splitk2=" << *e.splitk2_splits;
    if (key.b_f16)
      o << " bf16";
    o << "\n";
  }
  return o.str();
}

} // namespace tensor_ash
