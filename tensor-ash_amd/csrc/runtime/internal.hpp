// Internal declarations of the host runtime (not part of the public API).
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <optional>
#include <string>
#include <vector>

#include "../kernels/kernel_args.h"
#include "tensor_ash.hpp"

namespace tensor_ash {

[[noreturn]] void fail(const std::string &msg);
std::string fmt_shape(const std::vector<uint32_t> &shape); // "[a, b, c]"
void hip_check(hipError_t err, const char *what);

// Every device and pinned-host allocation the library makes goes through
// these two, which count the calls (allocation_count) so a caller can
// check that an entry point allocated nothing.
hipError_t device_malloc(void **ptr, size_t bytes);
hipError_t host_malloc(void **ptr, size_t bytes, unsigned int flags);
uint64_t allocation_count();

struct DeviceBuffer {
  std::shared_ptr<Context> ctx;
  void *ptr = nullptr;
  uint64_t bytes = 0;
  ~DeviceBuffer();
};

// src/matmul/resolution.rs:10-76.
struct MatrixShape {
  uint32_t batch, rows, cols;
  static MatrixShape from_tensor_shape(const std::vector<uint32_t> &shape);
  uint32_t batch_stride(const char *label) const;
};

// src/matmul/resolution.rs:80-442.
struct ResolvedMatmul {
  uint32_t m = 0, n = 0, k = 0, batch = 0;
  uint32_t batch_stride_a = 0, batch_stride_b = 0, batch_stride_c = 0;
  uint64_t total_flops = 0;
  bool b_f16 = false;
  bool a_f16 = false;
  bool packed_b = false;

  static ResolvedMatmul from_shapes(const std::vector<uint32_t> &a,
                                    const std::vector<uint32_t> &b,
                                    const std::vector<uint32_t> &c);
  static ResolvedMatmul from_call(const MatmulCall &call);
  static ResolvedMatmul from_op(const MatmulOp &op);
  void validate_bias_shape(const std::vector<uint32_t> &shape) const;
  void validate_epilogue(const MatmulOp &op) const;
  void validate_normed_a(const MatmulOp &op) const;
  void validate_store(const MatmulOp &op) const;
  bool operator==(const ResolvedMatmul &o) const;
};
uint64_t total_flops(const std::vector<ResolvedMatmul> &resolved);

// Largest rows a decode GEMV launch handles (register-resident X rows).
constexpr uint32_t kGemvMaxRows = 8;

// ---- routing (src/pipeline/mod.rs:293-535, selection.rs:89-172) ----
size_t heuristic_kernel_index(uint32_t cus, uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                              bool b_f16, bool packed_b, bool a_f16 = false);
bool kernel_supports(const KernelSpec &spec, const ResolvedMatmul &dims);
bool gemm_lds_ok(const ResolvedMatmul &dims);
bool f32_mi16_ok(const ResolvedMatmul &dims, uint32_t tile_m, uint32_t tile_n, uint32_t planes);
uint32_t mi16_threads(uint32_t tile_m);
bool f16_dual_tile(const KernelSpec &spec);
std::vector<size_t> tune_candidate_indices(const ResolvedMatmul &dims);
size_t registry_index(const char *name);

// ---- split-K (src/executor/splitk2.rs) ----
constexpr uint32_t kReduceThreads = 256;
constexpr uint64_t kAutoScratchCapBytes = 256ull << 20;
const KernelSpec &splitk_stage1_spec(uint32_t m, uint32_t n, uint32_t k);
uint32_t gemm_threads(const KernelSpec &s);
uint32_t h16sk_splits(uint32_t cus, uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                      uint32_t tile_m, uint32_t tile_n);
uint32_t splitk_sub_splits(uint32_t cus, const ResolvedMatmul &dims, uint32_t splits);
std::optional<uint32_t> heuristic_splits(uint32_t cus, uint32_t batch, uint32_t m, uint32_t n,
                                         uint32_t k);
uint32_t splitk_reduce_groups(uint32_t cus, uint64_t quads, uint32_t planes);
uint32_t default_num_k_splits(uint32_t cus, uint32_t batch, uint32_t m, uint32_t n, uint32_t k);
bool auto_route_fits(uint32_t batch, uint32_t m, uint32_t n, uint32_t k, uint32_t splits);
void validate_scratch_geometry(uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                               uint32_t splits);
std::optional<uint64_t> checked_auto_scratch_end(uint64_t offset, uint64_t bytes);

// ---- GEMV geometry ----
struct GemvPlan {
  uint32_t tw = 64, mr = 1, tiles = 0, kchunk = 0, kchunks = 1;
  uint64_t partial_bytes = 0; // 0 when kchunks == 1
};
uint32_t gemv_unit(uint32_t tw, bool f32_weights, bool dual, uint32_t rows);
GemvPlan plan_gemv(uint32_t cus, uint32_t rows, uint32_t n, uint32_t k, uint32_t tw, bool dual,
                   uint32_t unit);

// ---- f16w A conversions converted up front ----
// One op of a submission as the paired up-front conversion sees it: its A
// (buffer, device pointer, values converted), whether its route converts A
// to f16, and the buffers it writes.
struct CvtCandidate {
  const void *a_buffer = nullptr;
  const void *a_ptr = nullptr;
  uint64_t n = 0;
  bool converts = false;
  const void *writes[2] = {nullptr, nullptr};
};
// Indices of the ops whose A is converted at submission start: the first
// two distinct A's that take the conversion and that no earlier op writes
// (fewer than two: nothing is paired).
std::vector<size_t> paired_conversion_picks(const std::vector<CvtCandidate> &ops);

// ---- tuner (src/executor/tuning.rs:300-313, pipeline/tuning.rs) ----
std::optional<uint64_t> median(std::vector<uint64_t> samples);
size_t candidate_at(size_t len, uint32_t round, size_t offset);

struct TuneKey {
  uint32_t batch, m, n, k;
  bool b_f16;
  bool operator<(const TuneKey &o) const;
};
struct TuneEntry {
  size_t kernel;
  std::optional<uint32_t> splitk2_splits;
};
std::string tune_store_path(const Context &ctx);
std::string tune_header_line(const Context &ctx);
std::map<TuneKey, TuneEntry> parse_tune_store(const std::string &text, const std::string &header);
std::string format_tune_store(const std::map<TuneKey, TuneEntry> &map, const std::string &header);

// Fixed device scratch (fixed_scratch.hip): the array's address on
// `device` (the current device), resolved once per device, and the mutex
// that serialises its users on that device.
hipError_t fixed_scratch_address(int device, void **out);
std::mutex &fixed_scratch_mutex(int device);

} // namespace tensor_ash
