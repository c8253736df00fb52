// Host-runtime unit tests (no GPU).  Counterparts of the reference's Rust
// unit tests: src/matmul/tests.rs:4-165, src/pipeline/catalog.rs:384-493,
// src/executor/splitk2.rs:472-607, src/executor/tuning.rs:319-345,
// src/dtype.rs:114-164.  Built and run by tests/test_capi_cpu.py.
#include <cmath>
#include <cstdio>
#include <functional>
#include <set>
#include <string>
#include <vector>

#include "../../tensor-ash_amd/csrc/runtime/internal.hpp"

using namespace tensor_ash;

static int g_fail = 0, g_pass = 0;
#define CHECK(...)                                                                   \
  do {                                                                                \
    if (__VA_ARGS__)                                                                       \
      ++g_pass;                                                                       \
    else {                                                                            \
      ++g_fail;                                                                       \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #__VA_ARGS__);                   \
    }                                                                                 \
  } while (0)

static std::string error_of(const std::function<void()> &f) {
  try {
    f();
  } catch (const Error &e) {
    return e.what();
  }
  return "";
}
static bool has(const std::string &s, const char *sub) { return s.find(sub) != std::string::npos; }

static void test_resolution() {
  // tests.rs:4-22
  auto r = ResolvedMatmul::from_shapes({2, 3}, {3, 4}, {2, 4});
  CHECK(r.m == 2 && r.n == 4 && r.k == 3 && r.batch == 1);
  CHECK(r.batch_stride_a == 0 && r.batch_stride_b == 0 && r.batch_stride_c == 0);
  CHECK(r.total_flops == 48);
  // tests.rs:24-37
  r = ResolvedMatmul::from_shapes({5, 2, 3}, {5, 3, 4}, {5, 2, 4});
  CHECK(r.batch == 5 && r.batch_stride_a == 6 && r.batch_stride_b == 12 && r.batch_stride_c == 8);
  CHECK(r.total_flops == 240);
  // tests.rs:39-50
  auto a = ResolvedMatmul::from_shapes({1, 2, 3}, {7, 3, 4}, {7, 2, 4});
  auto b = ResolvedMatmul::from_shapes({7, 2, 3}, {1, 3, 4}, {7, 2, 4});
  auto both = ResolvedMatmul::from_shapes({1, 2, 3}, {1, 3, 4}, {7, 2, 4});
  CHECK(a.batch_stride_a == 0 && a.batch_stride_b == 12);
  CHECK(b.batch_stride_a == 6 && b.batch_stride_b == 0);
  CHECK(both.batch_stride_a == 0 && both.batch_stride_b == 0 && both.batch_stride_c == 8);
  CHECK(both.total_flops == 336);
  // tests.rs:52-78
  std::string e = error_of([] { ResolvedMatmul::from_shapes({2, 3}, {5, 4}, {2, 4}); });
  CHECK(has(e, "A.K=3") && has(e, "B.K=5"));
  e = error_of([] { ResolvedMatmul::from_shapes({7, 2, 3}, {7, 3, 4}, {1, 2, 4}); });
  CHECK(has(e, "incompatible batch dims") && has(e, "A.B=7"));
  e = error_of([] { MatrixShape::from_tensor_shape({0, 3}); });
  CHECK(has(e, "non-zero"));
  e = error_of([] { MatrixShape::from_tensor_shape({1, 2, 3, 4}); });
  CHECK(has(e, "rank 4"));
  // tests.rs:80-93
  e = error_of([] {
    ResolvedMatmul::from_shapes({2, UINT32_MAX, UINT32_MAX}, {1, UINT32_MAX, 1},
                                {2, UINT32_MAX, 1});
  });
  CHECK(has(e, "A batch stride") && has(e, "overflows"));
  // tests.rs:95-99
  CHECK(error_of([] { ResolvedMatmul::from_shapes({65536, 65536}, {65536, 1}, {65536, 1}); })
            .empty());
  CHECK(error_of([] {
          ResolvedMatmul::from_shapes({2, 32768, 65536}, {65536, 1}, {2, 32768, 1});
        }).empty());
  // tests.rs:101-125
  struct Case {
    const char *label;
    std::vector<uint32_t> a, b, c;
  } cases[] = {
      {"A", {65537, 65536}, {65536, 1}, {65537, 1}},
      {"B", {1, 65537}, {65537, 65536}, {1, 65536}},
      {"C", {65537, 1}, {1, 65536}, {65537, 65536}},
      {"A", {3, 32768, 65536}, {65536, 1}, {3, 32768, 1}},
      {"B", {3, 1, 32768}, {3, 32768, 65536}, {3, 1, 65536}},
      {"C", {3, 32768, 1}, {1, 65536}, {3, 32768, 65536}},
  };
  for (auto &cs : cases) {
    e = error_of([&] { ResolvedMatmul::from_shapes(cs.a, cs.b, cs.c); });
    CHECK(has(e, cs.label) && has(e, "shader u32 indexing"));
  }
  // tests.rs:127-134
  e = error_of([] { ResolvedMatmul::from_shapes({1, UINT32_MAX}, {UINT32_MAX, 1}, {UINT32_MAX, 1, 1}); });
  CHECK(has(e, "FLOP count overflows"));
  // tests.rs:136-145
  auto d = ResolvedMatmul::from_shapes({3, 2, 4}, {3, 4, 5}, {3, 2, 5});
  CHECK(error_of([&] { d.validate_bias_shape({5}); }).empty());
  CHECK(error_of([&] { d.validate_bias_shape({3, 5}); }).empty());
  CHECK(has(error_of([&] { d.validate_bias_shape({5, 3}); }), "bias shape"));
  // RunStats::tflops (tests.rs:152-165)
  RunStats s{1000000, 1, 2000000000};
  CHECK(s.tflops() && std::fabs(*s.tflops() - 2.0) < 1e-12);
  s.gpu_time_ns = 0;
  CHECK(!s.tflops());
  s.gpu_time_ns.reset();
  CHECK(!s.tflops());
}

static void test_registry() {
  // catalog.rs:384-417 / 483-493: unique names, every name and alias parses
  // case-insensitively with surrounding whitespace, "" / "auto" are Auto.
  std::set<std::string> names;
  for (size_t i = 0; i < KERNEL_SPECS_LEN; ++i) {
    CHECK(names.insert(KERNEL_SPECS[i].name).second);
    std::string up = KERNEL_SPECS[i].name;
    for (auto &c : up)
      c = (char)std::toupper((unsigned char)c);
    auto sel = KernelSelection::parse("  " + up + "  ");
    CHECK(sel.index && *sel.index == i);
  }
  CHECK(KernelSelection::parse("").is_auto() && KernelSelection::parse(" AUTO ").is_auto());
  CHECK(*KernelSelection::parse("large").index == registry_index("f32_m256n256"));
  CHECK(*KernelSelection::parse("row_bda").index == registry_index("f32_gemv_row"));
  CHECK(has(error_of([] { KernelSelection::parse("wideish"); }), "invalid ML_KERNEL 'wideish'"));
}

static void test_routing() {
  const uint32_t cus = 256;
  auto name = [&](uint32_t b, uint32_t m, uint32_t n, uint32_t k, bool f16, bool packed) {
    return std::string(KERNEL_SPECS[heuristic_kernel_index(cus, b, m, n, k, f16, packed)].name);
  };
  CHECK(name(1, 4096, 4096, 4096, false, false) == "f32_m256n256");
  CHECK(name(8, 2048, 2048, 2048, false, false) == "f32_m256n256");
  CHECK(name(1, 512, 512, 512, false, false) == "f32_m64n64");
  // config-5 prefill shapes (M = 512): QKV, O, gate/up, down
  CHECK(name(1, 512, 2560, 2048, true, false) == "f16w_mfma_m64n128");
  CHECK(name(1, 2560, 512, 2048, true, false) == "f16w_mfma_m128n64");
  CHECK(name(1, 512, 2048, 2048, true, false) == "f16w_mfma_m64n64");
  CHECK(name(1, 512, 5632, 2048, true, false) == "f16w_mfma_m128n128");
  CHECK(name(1, 512, 2048, 5632, true, false) == "f16w_sk_m128n128");
  CHECK(h16sk_splits(cus, 1, 512, 2048, 5632, 128, 64) == 2);
  CHECK(h16sk_splits(cus, 1, 512, 2048, 5632, 128, 128) == 4);
  CHECK(h16sk_splits(cus, 1, 4096, 4096, 4096, 64, 128) == 1);
  CHECK(name(1, 4096, 4096, 4096, true, false) == "f16w_mfma_m256n256");
  CHECK(name(1, 2048, 4096, 4096, true, false) == "f16w_mfma_m128n128");
  // Ragged K or N: register-staged tiles only (no 256x256).
  CHECK(name(1, 4096, 4096, 4000, true, false) == "f16w_mfma_m128n128");
  CHECK(name(1, 4096, 4100, 4096, true, false) == "f16w_mfma_m128n128");
  CHECK(name(1, 32, 4096, 4096, true, false) == "f16w_m64n64"); // M < 64: exact widening path
  CHECK(std::string(KERNEL_SPECS[heuristic_kernel_index(cus, 1, 512, 256, 2048, true, false, true)]
                        .name) == "f16w_a16_m64n64");
  CHECK(name(1, 1, 5632, 2048, true, true) == "f16w_gemv_packed_t64");
  CHECK(name(1, 8, 96, 2048, true, true) == "f16w_gemv_packed_t32");
  CHECK(name(1, 1, 4096, 4096, false, false) == "f32_gemv_row");
  CHECK(name(1, 8, 4096, 4096, true, false) == "f16w_gemv_row");
  CHECK(name(1, 9, 4096, 4096, true, false) != "f16w_gemv_row");
  CHECK(name(2, 1, 4096, 4096, false, false) != "f32_gemv_row");
  CHECK(name(1, 3, 998, 1000, true, false) == "f16w_m64n64"); // N % 4 != 0
  // every candidate the tuner measures can run the shape
  auto d = ResolvedMatmul::from_shapes({64, 300}, {300, 200}, {64, 200});
  for (size_t i : tune_candidate_indices(d))
    CHECK(kernel_supports(KERNEL_SPECS[i], d) && !KERNEL_SPECS[i].weights_f16());
  d.b_f16 = true;
  d.packed_b = true;
  CHECK(tune_candidate_indices(d).empty()); // M=64 > 8 rows: no packed route
}

static void test_splitk() {
  // Reduce plane groups: a power of two within [1, min(planes, 256)], a pure
  // function of the shape (fixed summation order), and more groups for
  // small outputs.
  CHECK(splitk_reduce_groups(256, 4096, 256) == 32);
  CHECK(splitk_reduce_groups(256, 1024, 256) == 64); // >= 4 planes per group
  CHECK(splitk_reduce_groups(256, 1024, 512) == 128);
  CHECK(splitk_reduce_groups(256, 1u << 20, 64) == 8);
  CHECK(splitk_reduce_groups(256, 16, 3) == 2);
  CHECK(splitk_reduce_groups(256, 16, 2) == 2);
  for (uint32_t planes : {2u, 3u, 7u, 8u, 100u, 256u, 4096u})
    for (uint64_t quads : {1ull, 100ull, 4096ull, 1ull << 22}) {
      const uint32_t g = splitk_reduce_groups(256, quads, planes);
      CHECK(g >= 1 && g <= planes && g <= 256 && (g & (g - 1)) == 0);
    }
  const uint32_t cus = 256;
  // Behaviour (targets are this build's own, for 256 CUs):
  // 4 tiles of 64x64, windows of whole pipeline loops: one WG per CU
  CHECK(heuristic_splits(cus, 1, 64, 256, 65536) == 64u);
  CHECK(heuristic_splits(cus, 1, 64, 256, 65536 + 64) == 128u); // unaligned: ~2 WGs per CU
  CHECK(heuristic_splits(cus, 1, 32, 128, 131072) == 128u);
  CHECK(heuristic_splits(cus, 1, 256, 256, 16384) == 16u);  // 64x64 pipelined stage 1: 16 tiles
  CHECK(std::string(splitk_stage1_spec(256, 256, 16384).name) == "f32_m64n64");
  CHECK(std::string(splitk_stage1_spec(256, 256, 16000).name) == "f32_m128n128");
  CHECK(heuristic_splits(cus, 1, 64, 64, 1024) == 4u);      // capped by K/256
  CHECK(!heuristic_splits(cus, 1, 64, 64, 512));            // K < 1024
  CHECK(!heuristic_splits(cus, 1, 4096, 4096, 4096));       // grid already full
  CHECK(!heuristic_splits(cus, 0, 64, 64, 4096));
  CHECK(!heuristic_splits(cus, 1, 1, 4096, 8192));
  CHECK(default_num_k_splits(cus, 1, 64, 64, 64) == 2);     // K / 32
  CHECK(default_num_k_splits(cus, 1, 4096, 4096, 4096) == 1);
  // splitk2.rs:515-520 (scratch geometry)
  CHECK(has(error_of([] { validate_scratch_geometry(1, 64, 64, 64, 65); }), "exceeds K=64"));
  CHECK(!error_of([] { validate_scratch_geometry(1, 65536, 65536, 2, 2); }).empty());
  CHECK(error_of([] { validate_scratch_geometry(1, 32768, 65536, 2, 2); }).empty());
  // splitk2.rs:559-595 (auto_route_fits, grid limits adapted to HIP)
  CHECK(auto_route_fits(1, 64, 64, 1024, 16));
  CHECK(!auto_route_fits(0, 64, 64, 1024, 16));
  CHECK(!auto_route_fits(1, 64, 64, 1024, 1));
  CHECK(!auto_route_fits(1, 64, 64, 65536, 65536));
  CHECK(!auto_route_fits(1, 64, 64, 8, 16));
  CHECK(!auto_route_fits(UINT32_MAX, UINT32_MAX, UINT32_MAX, UINT32_MAX, 2));
  CHECK(auto_route_fits(1, 1024, 1024, 4096, 64));  // exactly the 256 MiB budget
  CHECK(!auto_route_fits(1, 1024, 1025, 4096, 64));
  // splitk2.rs:597-606 (aligned, checked, capped reservation)
  CHECK(checked_auto_scratch_end(0, 1) == 16u);
  CHECK(checked_auto_scratch_end(kAutoScratchCapBytes - 16, 16) == kAutoScratchCapBytes);
  CHECK(!checked_auto_scratch_end(kAutoScratchCapBytes, 1));
  CHECK(!checked_auto_scratch_end(UINT64_MAX - 7, 8));
  CHECK(!checked_auto_scratch_end(0, UINT64_MAX));
}

static void test_gemv_plan() {
  for (uint32_t tw : {32u, 64u})
    for (bool f32w : {false, true})
      for (bool dual : {false, true})
        for (uint32_t rows : {1u, 3u, 8u})
          for (uint32_t k : {64u, 300u, 2048u, 5632u, 65536u}) {
            const uint32_t unit = gemv_unit(tw, f32w, dual, rows);
            CHECK(unit == 4 * (64 / (tw / (f32w ? 2 : 4))) * (rows > 2 ? 8 : 16));
            GemvPlan p = plan_gemv(256, rows, 5632, k, tw, dual, unit);
            CHECK(p.kchunk % unit == 0 && p.kchunk >= unit);
            CHECK((uint64_t)p.kchunk * p.kchunks >= k && (uint64_t)p.kchunk * (p.kchunks - 1) < k);
            CHECK(p.kchunk * p.mr <= 4096 || p.kchunk == unit); // fits the kernel's X window
            CHECK(p.mr >= rows && p.mr <= 8);
            CHECK(p.kchunks == 1 ? p.partial_bytes == 0
                                 : p.partial_bytes == (uint64_t)p.kchunks * p.tiles *
                                                          (dual ? 2 : 1) * p.mr * tw * 4);
          }
  // One row, at least one tile per CU: whole-K units (lm_head); fewer tiles
  // keep ~3 workgroups per CU.
  const uint32_t u1 = gemv_unit(64, false, false, 1);
  CHECK(plan_gemv(256, 1, 32000, 2048, 64, false, u1).kchunks == 1u);
  CHECK(plan_gemv(256, 1, 5632, 2048, 64, false, u1).kchunks == 8u);
  CHECK(plan_gemv(256, 4, 32000, 2048, 64, false, gemv_unit(64, false, false, 4)).kchunks > 1u);
}

static void test_tuner_helpers() {
  // tuning.rs:319-345
  CHECK(!median({}));
  CHECK(median({9, 1, 5}) == 5u);
  CHECK(median({8, 2}) == 5u);
  for (uint32_t round = 0; round <= 4; ++round) {
    std::vector<size_t> order;
    for (size_t off = 0; off < 19; ++off)
      order.push_back(candidate_at(19, round, off));
    std::sort(order.begin(), order.end());
    for (size_t i = 0; i < 19; ++i)
      CHECK(order[i] == i);
  }
  for (uint32_t rounds : {2u, 4u}) {
    std::vector<size_t> rank_sums(19, 0);
    for (uint32_t round = 1; round <= rounds; ++round)
      for (size_t rank = 0; rank < 19; ++rank)
        rank_sums[candidate_at(19, round, rank)] += rank;
    for (size_t v : rank_sums)
      CHECK(v == rank_sums[0]);
  }
  // tune store: round trip, header binding, malformed lines skipped
  std::map<TuneKey, TuneEntry> m;
  m[TuneKey{1, 64, 256, 65536, false}] = TuneEntry{registry_index("f32_m64n64"), 32u};
  m[TuneKey{1, 512, 2560, 2048, true}] = TuneEntry{registry_index("f16w_m64n64"), std::nullopt};
  const std::string hdr = "tensor-ash-tune-v3 hip=1 arch=gfx950 kernels=00000000000000ab";
  std::string text = format_tune_store(m, hdr);
  auto back = parse_tune_store(text + "garbage line\n1 2 3\n1 1 1 1 no_such_kernel\n0 1 1 1 f32_m64n64\n"
                                      "1 8 8 8 f32_m64n64 splitk2=1\n",
                               hdr);
  CHECK(back.size() == 3);
  CHECK(back[TuneKey{1, 64, 256, 65536, false}].splitk2_splits == 32u);
  CHECK(back[TuneKey{1, 512, 2560, 2048, true}].kernel == registry_index("f16w_m64n64"));
  CHECK(!back[TuneKey{1, 8, 8, 8, false}].splitk2_splits); // splitk2=1 is out of range
  CHECK(parse_tune_store(text, hdr + "x").empty());
}

static void test_dtype() {
  // dtype.rs:118-163
  CHECK(f32_to_f16_bits(1.0f) == 0x3c00 && f32_to_f16_bits(-2.0f) == 0xc000);
  CHECK(f32_to_f16_bits(65504.0f) == 0x7bff && f32_to_f16_bits(65520.0f) == 0x7c00);
  CHECK(f32_to_f16_bits(INFINITY) == 0x7c00);
  CHECK(f32_to_f16_bits(6.104e-5f) == 0x0400 && f32_to_f16_bits(5.96e-8f) == 0x0001);
  CHECK(f32_to_f16_bits(1e-10f) == 0);
  CHECK(std::isnan(f16_bits_to_f32(f32_to_f16_bits(NAN))));
  CHECK(round_f32_via_f16(1.0f + std::ldexp(1.0f, -11)) == 1.0f);
  CHECK(round_f32_via_f16(1.0f + 3 * std::ldexp(1.0f, -11)) == 1.0f + std::ldexp(1.0f, -9));
  // subnormal halves decode exactly: 0x0001 = 2^-24, 0x0200 = 2^-15
  CHECK(f16_bits_to_f32(0x0001) == std::ldexp(1.0f, -24));
  CHECK(f16_bits_to_f32(0x0200) == std::ldexp(1.0f, -15));
  CHECK(f16_bits_to_f32(0x83ff) == -1023 * std::ldexp(1.0f, -24));
  for (uint32_t h = 0; h < 65536; ++h) {
    const float f = f16_bits_to_f32((uint16_t)h);
    if (!std::isnan(f))
      CHECK(f32_to_f16_bits(f) == h); // exact round trip of every half
  }
  // api.rs:355-380
  float src[16];
  for (int i = 0; i < 16; ++i)
    src[i] = (float)i;
  auto p = pack_f16w_row_tiles(src, 4, 4, 2);
  const float want[16] = {0, 1, 4, 5, 8, 9, 12, 13, 2, 3, 6, 7, 10, 11, 14, 15};
  for (int i = 0; i < 16; ++i)
    CHECK(p[i] == want[i]);
  CHECK(has(error_of([&] { pack_f16w_row_tiles(src, 4, 4, 3); }), "not a multiple of tile_n=3"));
}

static void test_paired_conversion_picks() {
  // The f16w route's up-front conversion pairs the first two distinct A's
  // that are converted and that no earlier op of the submission writes.
  int x, y, z, a2, c0, c1, c2, c3;
  auto op = [](const void *a, bool conv, const void *c, uint64_t n = 100) {
    CvtCandidate k;
    k.a_buffer = a;
    k.a_ptr = a;
    k.n = n;
    k.converts = conv;
    k.writes[0] = c;
    return k;
  };
  using V = std::vector<size_t>;
  // the prefill layer: QKV(x), O(attn), up(x), gate(x), down(h from gate)
  CHECK(paired_conversion_picks({op(&x, true, &c0), op(&a2, true, &c1), op(&x, true, &c2),
                                 op(&x, true, &y), op(&y, true, &c3)}) == V{0, 1});
  // a repeated A is not paired with itself
  CHECK(paired_conversion_picks({op(&x, true, &c0), op(&x, true, &c1), op(&a2, true, &c2)}) ==
        V{0, 2});
  // an A an earlier op writes is skipped (converted when its op runs)
  CHECK(paired_conversion_picks({op(&x, true, &y), op(&y, true, &c0), op(&a2, true, &c1),
                                 op(&x, true, &c2)}) == V{0, 2});
  CHECK(paired_conversion_picks({op(&a2, true, &x), op(&x, true, &c0), op(&z, true, &c1)}) ==
        V{0, 2});
  // a store destination counts as written too
  {
    auto w = op(&c0, false, &c1);
    w.writes[1] = &x;
    CHECK(paired_conversion_picks({w, op(&x, true, &c2), op(&a2, true, &c3), op(&z, true, &y)}) ==
          V{2, 3});
  }
  // ops whose route does not convert A are ignored
  CHECK(paired_conversion_picks({op(&x, false, &c0), op(&a2, true, &c1), op(&z, true, &c2)}) ==
        V{1, 2});
  // the same buffer viewed with a different element count is a distinct copy
  CHECK(paired_conversion_picks({op(&x, true, &c0, 100), op(&x, true, &c1, 200)}) == V{0, 1});
  // fewer than two candidates: nothing paired
  CHECK(paired_conversion_picks({op(&x, true, &c0), op(&x, true, &c1)}).empty());
  CHECK(paired_conversion_picks({op(&x, true, &c0), op(&a2, false, &c1)}).empty());
  CHECK(paired_conversion_picks({}).empty());
}

int main() {
  test_resolution();
  test_registry();
  test_routing();
  test_splitk();
  test_gemv_plan();
  test_tuner_helpers();
  test_dtype();
  test_paired_conversion_picks();
  std::printf("%d checks, %d failed\n", g_pass + g_fail, g_fail);
  if (g_fail == 0)
    std::printf("all passed\n");
  return g_fail ? 1 : 0;
}
