// vendor_bench: FP32 SGEMM of the vendor library (hipBLASLt), timed with
// HIP events on the GPU only, as the comparison baseline for the fused GEMM
// path (the role of the reference's benchmarks/cublas_bench/cublas_bench.cu:
// same CSV in / CSV out contract, cublas_bench.cu:30-45).
//
//   vendor_bench [--iters N] [--warmup N] [--algos N] < cases.csv
//
// stdin:  label,b,m,n,k            (header line optional)
// stdout: label,b,m,n,k,best_ms,mean_ms,tflops,sample_count,min_ms,median_ms,p95_ms,algo
//
// Row-major C[M,N] = A[M,K] @ B[K,N] is computed as the column-major
// product C^T = B^T A^T (no transposes: hipBLASLt sees B as an N x K
// column-major matrix with ld N).  Compute type is HIPBLAS_COMPUTE_32F
// (full FP32; the library has no reduced-precision fallback on this type).
// The --algos best heuristic candidates are each timed and the fastest is
// reported, so the baseline is the library at its best, not its default.
// tflops uses the median.  Inputs are uniform [-1, 1) from a fixed LCG.

#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

namespace {

void hip_ok(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "vendor_bench: %s: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}
void blas_ok(hipblasStatus_t s, const char *what) {
  if (s != HIPBLAS_STATUS_SUCCESS) {
    std::fprintf(stderr, "vendor_bench: %s: hipblas status %d\n", what, (int)s);
    std::exit(1);
  }
}

struct Case {
  std::string label;
  long long b = 1, m = 0, n = 0, k = 0;
};

std::vector<Case> read_cases() {
  std::vector<Case> out;
  std::string line;
  while (std::getline(std::cin, line)) {
    if (line.empty() || line[0] == '#' || line.rfind("label", 0) == 0)
      continue;
    std::stringstream ss(line);
    Case c;
    std::string f;
    std::getline(ss, c.label, ',');
    long long *dims[] = {&c.b, &c.m, &c.n, &c.k};
    for (long long *d : dims) {
      if (!std::getline(ss, f, ',')) {
        std::fprintf(stderr, "vendor_bench: bad case line '%s'\n", line.c_str());
        std::exit(2);
      }
      *d = std::atoll(f.c_str());
    }
    if (c.b < 1 || c.m < 1 || c.n < 1 || c.k < 1) {
      std::fprintf(stderr, "vendor_bench: nonpositive dimension in '%s'\n", line.c_str());
      std::exit(2);
    }
    out.push_back(c);
  }
  return out;
}

void fill_uniform(std::vector<float> &v, uint64_t seed) {
  uint64_t s = seed * 0x9E3779B97F4A7C15ull | 1ull;
  for (float &x : v) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    x = (float)((s >> 40) & 0xFFFFFF) / 16777216.0f * 2.0f - 1.0f;
  }
}

struct Layouts {
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  ~Layouts() {
    if (a)
      hipblasLtMatrixLayoutDestroy(a);
    if (b)
      hipblasLtMatrixLayoutDestroy(b);
    if (c)
      hipblasLtMatrixLayoutDestroy(c);
  }
};

hipblasLtMatrixLayout_t layout(long long rows, long long cols, long long ld, long long batch,
                               long long stride) {
  hipblasLtMatrixLayout_t l = nullptr;
  blas_ok(hipblasLtMatrixLayoutCreate(&l, HIP_R_32F, rows, cols, ld), "MatrixLayoutCreate");
  if (batch > 1) {
    const int32_t bc = (int32_t)batch;
    const int64_t st = stride;
    blas_ok(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc,
                                              sizeof(bc)),
            "layout batch count");
    blas_ok(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &st,
                                              sizeof(st)),
            "layout batch stride");
  }
  return l;
}

} // namespace

int main(int argc, char **argv) {
  int iters = 30, warmup = 8, algos = 8;
  for (int i = 1; i < argc; ++i) {
    auto next = [&]() -> int {
      if (i + 1 >= argc) {
        std::fprintf(stderr, "vendor_bench: %s needs a value\n", argv[i]);
        std::exit(2);
      }
      return std::atoi(argv[++i]);
    };
    if (!std::strcmp(argv[i], "--iters"))
      iters = next();
    else if (!std::strcmp(argv[i], "--warmup"))
      warmup = next();
    else if (!std::strcmp(argv[i], "--algos"))
      algos = next();
    else {
      std::fprintf(stderr, "usage: vendor_bench [--iters N] [--warmup N] [--algos N] < cases.csv\n");
      return 2;
    }
  }
  if (iters < 1 || warmup < 0 || algos < 1) {
    std::fprintf(stderr, "vendor_bench: iters >= 1, warmup >= 0, algos >= 1\n");
    return 2;
  }
  const std::vector<Case> cases = read_cases();

  hipblasLtHandle_t handle = nullptr;
  blas_ok(hipblasLtCreate(&handle), "hipblasLtCreate");
  hipStream_t stream = nullptr;
  hip_ok(hipStreamCreate(&stream), "hipStreamCreate");
  hipEvent_t e0, e1;
  hip_ok(hipEventCreate(&e0), "hipEventCreate");
  hip_ok(hipEventCreate(&e1), "hipEventCreate");
  const uint64_t ws_bytes = 64ull << 20;
  void *ws = nullptr;
  hip_ok(hipMalloc(&ws, ws_bytes), "hipMalloc workspace");

  std::printf("label,b,m,n,k,best_ms,mean_ms,tflops,sample_count,min_ms,median_ms,p95_ms,algo\n");
  for (const Case &c : cases) {
    const size_t na = (size_t)(c.b * c.m * c.k), nb = (size_t)(c.b * c.k * c.n),
                 nc = (size_t)(c.b * c.m * c.n);
    std::vector<float> ha(na), hb(nb);
    fill_uniform(ha, 1);
    fill_uniform(hb, 2);
    float *da = nullptr, *db = nullptr, *dc = nullptr;
    hip_ok(hipMalloc(&da, na * 4), "hipMalloc A");
    hip_ok(hipMalloc(&db, nb * 4), "hipMalloc B");
    hip_ok(hipMalloc(&dc, nc * 4), "hipMalloc C");
    hip_ok(hipMemcpy(da, ha.data(), na * 4, hipMemcpyHostToDevice), "upload A");
    hip_ok(hipMemcpy(db, hb.data(), nb * 4, hipMemcpyHostToDevice), "upload B");

    hipblasLtMatmulDesc_t desc = nullptr;
    blas_ok(hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "MatmulDescCreate");
    // Column-major view: first operand B^T (n x k, ld n), second A^T (k x m, ld k).
    Layouts L;
    L.a = layout(c.n, c.k, c.n, c.b, c.k * c.n);
    L.b = layout(c.k, c.m, c.k, c.b, c.m * c.k);
    L.c = layout(c.n, c.m, c.n, c.b, c.m * c.n);
    hipblasLtMatmulPreference_t pref = nullptr;
    blas_ok(hipblasLtMatmulPreferenceCreate(&pref), "PreferenceCreate");
    blas_ok(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                  &ws_bytes, sizeof(ws_bytes)),
            "preference workspace");
    std::vector<hipblasLtMatmulHeuristicResult_t> heur(algos);
    int found = 0;
    blas_ok(hipblasLtMatmulAlgoGetHeuristic(handle, desc, L.a, L.b, L.c, L.c, pref, algos,
                                            heur.data(), &found),
            "AlgoGetHeuristic");
    if (found < 1) {
      std::fprintf(stderr, "vendor_bench: no algorithm for %s\n", c.label.c_str());
      return 1;
    }
    const float alpha = 1.0f, beta = 0.0f;
    auto run = [&](int a) {
      blas_ok(hipblasLtMatmul(handle, desc, &alpha, db, L.a, da, L.b, &beta, dc, L.c, dc, L.c,
                              &heur[a].algo, ws, ws_bytes, stream),
              "hipblasLtMatmul");
    };
    auto sample = [&](int a) {
      hip_ok(hipEventRecord(e0, stream), "hipEventRecord");
      run(a);
      hip_ok(hipEventRecord(e1, stream), "hipEventRecord");
      hip_ok(hipEventSynchronize(e1), "hipEventSynchronize");
      float ms = 0.f;
      hip_ok(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
      return (double)ms;
    };
    // Pick the fastest candidate on a short median, then time it fully.
    int best_algo = 0;
    double best_med = 1e300;
    for (int a = 0; a < found; ++a) {
      if (heur[a].state != HIPBLAS_STATUS_SUCCESS || heur[a].workspaceSize > ws_bytes)
        continue;
      for (int w = 0; w < 2; ++w)
        run(a);
      std::vector<double> t;
      for (int s = 0; s < 5; ++s)
        t.push_back(sample(a));
      std::sort(t.begin(), t.end());
      if (t[2] < best_med) {
        best_med = t[2];
        best_algo = a;
      }
    }
    for (int w = 0; w < warmup; ++w)
      run(best_algo);
    hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
    std::vector<double> ms;
    double sum = 0.0;
    for (int i = 0; i < iters; ++i) {
      ms.push_back(sample(best_algo));
      sum += ms.back();
    }
    std::sort(ms.begin(), ms.end());
    const size_t cnt = ms.size();
    const double median = cnt % 2 ? ms[cnt / 2] : 0.5 * (ms[cnt / 2 - 1] + ms[cnt / 2]);
    const double p95 = ms[std::min(cnt - 1, (size_t)(0.95 * (double)(cnt - 1) + 0.5))];
    const double flops = 2.0 * (double)c.b * (double)c.m * (double)c.n * (double)c.k;
    std::printf("%s,%lld,%lld,%lld,%lld,%.6f,%.6f,%.3f,%zu,%.6f,%.6f,%.6f,%d\n", c.label.c_str(),
                c.b, c.m, c.n, c.k, ms.front(), sum / (double)cnt, flops / (median * 1e-3) / 1e12,
                cnt, ms.front(), median, p95, best_algo);
    std::fflush(stdout);
    hipblasLtMatmulPreferenceDestroy(pref);
    hipblasLtMatmulDescDestroy(desc);
    hip_ok(hipFree(da), "hipFree");
    hip_ok(hipFree(db), "hipFree");
    hip_ok(hipFree(dc), "hipFree");
  }
  hip_ok(hipFree(ws), "hipFree workspace");
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  hipStreamDestroy(stream);
  hipblasLtDestroy(handle);
  return 0;
}
