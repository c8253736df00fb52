// Cross-workgroup hand-off latency probe (a measurement tool, not part of
// the library).  The persistent decode-MLP launch passes each layer through
// four hand-offs: a producer workgroup stores a value with an agent-scope
// store and a consumer workgroup polls for it.  This program measures that
// primitive as a ping-pong round trip between two workgroups, on an idle
// GPU and while a second kernel on another stream (default priority) reads
// HBM with every CU, the condition the decode chain's hand-offs run under.
//
// Producers always store with agent-scope vector stores.  Consumers poll
// with agent-scope vector loads (the decode kernel's form) or with scalar
// loads that miss the scalar cache (the `glc` form).  Workgroups 0 and 1 run
// on different XCDs (consecutive dispatch ids are dealt to the 8 XCDs in
// turn), 0 and 8 on the same one.  Every poll is bounded: a lost value is
// reported as a failure, never a hang.
//
//   lib/handoff_probe            (built by build.py with hipcc for gfx950)
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#define CK(x)                                                                           \
  do {                                                                                  \
    hipError_t e_ = (x);                                                                \
    if (e_ != hipSuccess) {                                                             \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                      \
      std::exit(1);                                                                     \
    }                                                                                   \
  } while (0)

namespace {

constexpr uint32_t kRounds = 1000;
constexpr uint32_t kPollLimit = 200000; // polls per round before giving up

enum Poll { kVector = 0, kScalar = 1 };

template <int POLL> __device__ __forceinline__ uint32_t poll(const uint32_t *p) {
  if constexpr (POLL == kVector) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    uint32_t v;
    asm volatile("s_load_dword %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
  }
}

// Workgroups a and b bounce the round number: a stores it to f0 and waits
// for it in f1, b waits for it in f0 and stores it to f1.  out = {elapsed
// ticks of a (100 MHz clock), failures of a, failures of b}.
template <int POLL>
__global__ void pingpong(uint32_t *f, uint32_t a, uint32_t b, uint64_t *out) {
  const uint32_t id = blockIdx.x;
  if ((id != a && id != b) || threadIdx.x != 0)
    return;
  uint32_t *f0 = f, *f1 = f + 64; // separate 256-byte lines
  uint32_t fails = 0;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (uint32_t i = 1; i <= kRounds && fails == 0; ++i) {
    if (id == a)
      __hip_atomic_store(f0, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t *src = id == a ? f1 : f0;
    uint32_t n = 0;
    while (poll<POLL>(src) != i)
      if (++n >= kPollLimit) {
        ++fails;
        break;
      }
    if (id == b && fails == 0)
      __hip_atomic_store(f1, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
  if (id == a) {
    out[0] = t1 - t0;
    out[1] = fails;
  } else {
    out[2] = fails;
  }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ void stream_read(const f32x4 *src, uint64_t n, float *sink, int reps) {
  float acc = 0.f;
  for (int r = 0; r < reps; ++r)
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
      const f32x4 v = __builtin_nontemporal_load(src + i);
      acc += v.x + v.y + v.z + v.w;
    }
  if (acc == 12345.f)
    sink[0] = acc;
}

struct Bufs {
  uint32_t *flags;
  uint64_t *out;
  f32x4 *big;
  float *sink;
  uint64_t n;
  hipStream_t s1, s2;
};

template <int POLL> void run(const Bufs &b, const char *poll_name, uint32_t wa, uint32_t wb, bool load) {
  CK(hipMemset(b.flags, 0, 4096));
  CK(hipMemset(b.out, 0, 64));
  CK(hipDeviceSynchronize());
  hipLaunchKernelGGL(pingpong<POLL>, dim3(16), dim3(64), 0, b.s1, b.flags, wa, wb, b.out);
  CK(hipGetLastError());
  if (load) {
    hipLaunchKernelGGL(stream_read, dim3(4096), dim3(256), 0, b.s2, b.big, b.n, b.sink, 40);
    CK(hipGetLastError());
  }
  CK(hipDeviceSynchronize());
  uint64_t h[3];
  CK(hipMemcpy(h, b.out, sizeof h, hipMemcpyDeviceToHost));
  std::printf("poll=%-6s workgroups=%u,%u %-8s %-13s round_trip_us=%.3f failures=%llu/%llu\n", poll_name,
              wa, wb, wb == 8 ? "same_xcd" : "two_xcds", load ? "under_stream" : "idle",
              h[0] * 0.01 / kRounds, (unsigned long long)h[1], (unsigned long long)h[2]);
}

} // namespace

int main() {
  Bufs b{};
  b.n = (2ull << 30) / sizeof(f32x4); // 2 GiB read per pass
  CK(hipMalloc(&b.flags, 4096));
  CK(hipMalloc(&b.out, 64));
  CK(hipMalloc(&b.big, b.n * sizeof(f32x4)));
  CK(hipMalloc(&b.sink, 4));
  CK(hipMemset(b.big, 0, b.n * sizeof(f32x4)));
  CK(hipStreamCreate(&b.s1));
  CK(hipStreamCreate(&b.s2));

  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  CK(hipEventRecord(e0, b.s2));
  hipLaunchKernelGGL(stream_read, dim3(4096), dim3(256), 0, b.s2, b.big, b.n, b.sink, 6);
  CK(hipEventRecord(e1, b.s2));
  CK(hipEventSynchronize(e1));
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, e0, e1));
  std::printf("read_stream_alone GB/s=%.1f\n", 6.0 * b.n * sizeof(f32x4) / ms / 1e6);

  for (int load = 0; load < 2; ++load)
    for (uint32_t wb : {1u, 8u}) {
      run<kVector>(b, "vector", 0, wb, load != 0);
      run<kScalar>(b, "scalar", 0, wb, load != 0);
    }
  CK(hipFree(b.flags));
  CK(hipFree(b.out));
  CK(hipFree(b.big));
  CK(hipFree(b.sink));
  return 0;
}
