// HIP device context, code-object loading and tensor storage.
// Replaces src/context/ and src/buffer.rs / src/tensor.rs allocation.
#include <atomic>
#include <dirent.h>
#include <dlfcn.h>

#include <algorithm>
#include <cctype>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <sstream>

#include "internal.hpp"

namespace tensor_ash {

void fail(const std::string &msg) { throw Error(msg); }

void hip_check(hipError_t err, const char *what) {
  if (err != hipSuccess)
    fail(std::string(what) + " failed: " + hipGetErrorString(err));
}

namespace {
std::atomic<uint64_t> g_allocations{0};
} // namespace

hipError_t device_malloc(void **ptr, size_t bytes) {
  g_allocations.fetch_add(1, std::memory_order_relaxed);
  return hipMalloc(ptr, bytes);
}

hipError_t host_malloc(void **ptr, size_t bytes, unsigned int flags) {
  g_allocations.fetch_add(1, std::memory_order_relaxed);
  return hipHostMalloc(ptr, bytes, flags);
}

uint64_t allocation_count() { return g_allocations.load(std::memory_order_relaxed); }

namespace {

// Directory of the code objects: $TA_KERNEL_DIR, else "kernels/" next to
// this shared library.
std::string kernel_dir() {
  if (const char *d = std::getenv("TA_KERNEL_DIR"); d && *d)
    return d;
  Dl_info info{};
  if (dladdr(reinterpret_cast<void *>(&kernel_dir), &info) && info.dli_fname) {
    std::string p = info.dli_fname;
    const size_t slash = p.rfind('/');
    return (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) + "/kernels";
  }
  return "kernels";
}

std::string lower(std::string s) {
  for (auto &c : s)
    c = (char)std::tolower((unsigned char)c);
  return s;
}

// src/context/device.rs:18-54 preference grammar, mapped onto HIP devices
// (every HIP device is a discrete GPU here).
int select_device(const std::string &raw_pref, int count) {
  std::string pref = raw_pref;
  pref.erase(0, pref.find_first_not_of(" \t\n"));
  pref.erase(pref.find_last_not_of(" \t\n") + 1);
  const std::string lc = lower(pref);
  if (lc.empty() || lc == "auto" || lc == "discrete")
    return 0;
  if (lc == "integrated" || lc == "virtual" || lc == "cpu")
    fail("no HIP device matches ML_DEVICE=" + lc + " (HIP devices are discrete GPUs)");
  auto parse_index = [&](const std::string &s) -> int {
    char *end = nullptr;
    const long v = std::strtol(s.c_str(), &end, 10);
    if (s.empty() || !end || *end != 0 || v < 0)
      fail("invalid ML_DEVICE index: " + s);
    if (v >= count)
      fail("no HIP device matches ML_DEVICE=index:" + s + " (" + std::to_string(count) +
           " available)");
    return (int)v;
  };
  if (lc.rfind("index:", 0) == 0)
    return parse_index(lc.substr(6));
  std::string name = lc;
  if (lc.rfind("name:", 0) == 0) {
    name = lower(pref.substr(5));
    name.erase(0, name.find_first_not_of(" \t"));
    name.erase(name.find_last_not_of(" \t") + 1);
    if (name.empty())
      fail("ML_DEVICE name filter must not be empty");
  } else if (!lc.empty() && std::all_of(lc.begin(), lc.end(), ::isdigit)) {
    return parse_index(lc);
  }
  for (int i = 0; i < count; ++i) {
    hipDeviceProp_t p{};
    if (hipGetDeviceProperties(&p, i) == hipSuccess &&
        (lower(p.name).find(name) != std::string::npos ||
         lower(p.gcnArchName).find(name) != std::string::npos))
      return i;
  }
  fail("no HIP device matches ML_DEVICE=name contains '" + name + "'");
}

} // namespace

std::shared_ptr<Context> Context::create(bool /*enable_validation*/,
                                         const std::string &preference) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    fail("no HIP device available");
  std::shared_ptr<Context> ctx(new Context());
  ctx->device_ = select_device(preference, count);
  hip_check(hipSetDevice(ctx->device_), "hipSetDevice");
  hipDeviceProp_t props{};
  hip_check(hipGetDeviceProperties(&props, ctx->device_), "hipGetDeviceProperties");
  ctx->cu_count_ = (uint32_t)props.multiProcessorCount;
  ctx->name_ = props.name;
  ctx->arch_ = props.gcnArchName;
  hip_check(hipRuntimeGetVersion(&ctx->runtime_version_), "hipRuntimeGetVersion");
  if (ctx->arch_.rfind("gfx950", 0) != 0)
    fail("tensor-ash kernels are built for gfx950 (MI355X); device " +
         std::to_string(ctx->device_) + " is " + ctx->arch_);

  // Load every code object; FNV-1a over their bytes keys the tune store.
  const std::string dir = kernel_dir();
  std::vector<std::string> files;
  if (DIR *d = opendir(dir.c_str())) {
    while (dirent *e = readdir(d)) {
      const std::string n = e->d_name;
      if (n.size() > 6 && n.substr(n.size() - 6) == ".hsaco")
        files.push_back(dir + "/" + n);
    }
    closedir(d);
  }
  std::sort(files.begin(), files.end());
  if (files.empty())
    fail("no gfx950 code objects (*.hsaco) found in " + dir +
         " (build them with __graft_entry__.build())");
  uint64_t h = 0xcbf29ce484222325ull;
  for (const auto &f : files) {
    std::ifstream in(f, std::ios::binary);
    std::vector<char> bytes((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    for (char c : bytes) {
      h ^= (uint8_t)c;
      h *= 0x100000001b3ull;
    }
    hipModule_t mod = nullptr;
    hip_check(hipModuleLoadData(&mod, bytes.data()), ("hipModuleLoadData " + f).c_str());
    ctx->modules_.push_back(mod);
  }
  ctx->code_hash_ = h;
  return ctx;
}

Context::~Context() {
  if (hipSetDevice(device_) == hipSuccess)
    for (void *m : modules_)
      (void)hipModuleUnload(static_cast<hipModule_t>(m));
}

void Context::make_current() const { hip_check(hipSetDevice(device_), "hipSetDevice"); }

void *Context::function(const std::string &symbol) const {
  static std::mutex mu;
  std::lock_guard<std::mutex> lock(mu);
  auto &fns = const_cast<std::vector<std::pair<std::string, void *>> &>(functions_);
  for (const auto &[name, f] : fns)
    if (name == symbol)
      return f;
  // A miss in one code object sets HIP's thread-local last error; clear it
  // again (unless an error was already pending) so the probe leaves no
  // trace for the host application's own error checks.
  const bool clean = hipPeekAtLastError() == hipSuccess;
  for (void *m : modules_) {
    hipFunction_t f = nullptr;
    const hipError_t e = hipModuleGetFunction(&f, static_cast<hipModule_t>(m), symbol.c_str());
    if (e != hipSuccess && clean)
      (void)hipGetLastError();
    if (e == hipSuccess && f) {
      fns.emplace_back(symbol, f);
      return f;
    }
  }
  fail("kernel symbol '" + symbol + "' not found in the loaded code objects");
}

DeviceBuffer::~DeviceBuffer() {
  if (ptr && ctx && hipSetDevice(ctx->device()) == hipSuccess)
    (void)hipFree(ptr);
}

// src/tensor.rs:35-52.
uint64_t Tensor::numel_checked(const std::vector<uint32_t> &shape) {
  if (shape.empty())
    fail("tensor shape must have at least one dimension");
  uint64_t acc = 1;
  for (size_t i = 0; i < shape.size(); ++i) {
    if (shape[i] == 0)
      fail("tensor dimension " + std::to_string(i) + " must be non-zero");
    if (acc > UINT64_MAX / shape[i])
      fail("tensor element count overflows u64");
    acc *= shape[i];
  }
  return acc;
}

// src/tensor.rs:57-92: device-resident, uninitialised; the byte size is
// rounded up to 16 so vector loads never leave the allocation.
Tensor Tensor::uninit_device(const std::shared_ptr<Context> &ctx,
                             const std::vector<uint32_t> &shape) {
  const uint64_t n = numel_checked(shape);
  if (n > UINT64_MAX / 4)
    fail("tensor byte size overflows u64");
  auto buf = std::make_shared<DeviceBuffer>();
  buf->ctx = ctx;
  buf->bytes = (n * 4 + 15) / 16 * 16;
  ctx->make_current();
  hip_check(device_malloc(&buf->ptr, buf->bytes), "hipMalloc");
  return Tensor(shape, DType::F32, buf);
}

Tensor Tensor::uninit_device_f16(const std::shared_ptr<Context> &ctx,
                                 const std::vector<uint32_t> &shape) {
  const uint64_t n = numel_checked(shape);
  if (n > UINT64_MAX / 2)
    fail("tensor byte size overflows u64");
  auto buf = std::make_shared<DeviceBuffer>();
  buf->ctx = ctx;
  buf->bytes = (n * 2 + 15) / 16 * 16;
  ctx->make_current();
  hip_check(device_malloc(&buf->ptr, buf->bytes), "hipMalloc");
  return Tensor(shape, DType::F16, buf);
}

// src/tensor.rs:98-117.
Tensor Tensor::alias_with_shape(const std::vector<uint32_t> &shape) const {
  const uint64_t n = numel_checked(shape);
  if (n != len()) {
    std::ostringstream o;
    o << "alias_with_shape: " << n << " elements for shape [";
    for (size_t i = 0; i < shape.size(); ++i)
      o << (i ? ", " : "") << shape[i];
    o << "] != " << len();
    fail(o.str());
  }
  return Tensor(shape, dtype_, buffer_);
}

uint64_t Tensor::len() const {
  uint64_t n = 1;
  for (uint32_t d : shape_)
    n *= d;
  return n;
}
uint64_t Tensor::size_bytes() const { return len() * dtype_size(dtype_); }
void *Tensor::device_ptr() const { return buffer_->ptr; }
bool Tensor::belongs_to(const Context *ctx) const { return buffer_->ctx.get() == ctx; }

// src/executor/cells.rs:163-205 (create_pos_buffer / create_host_u32_buffer
// / create_token_id_buffer): pinned, mapped host memory, zero-filled.
std::unique_ptr<U32Cell> U32Cell::create(const std::shared_ptr<Context> &ctx, uint32_t cap) {
  if (!ctx)
    fail("create_u32_cell: null context");
  if (cap == 0)
    fail("create_token_id_buffer: cap must be non-zero");
  ctx->make_current();
  std::unique_ptr<U32Cell> c(new U32Cell());
  void *host = nullptr;
  hip_check(host_malloc(&host, (size_t)cap * 4, hipHostMallocMapped), "hipHostMalloc (u32 cell)");
  void *dev = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&dev, host, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(host);
    hip_check(e, "hipHostGetDevicePointer (u32 cell)");
  }
  std::memset(host, 0, (size_t)cap * 4);
  c->ctx_ = ctx;
  c->host_ = static_cast<uint32_t *>(host);
  c->device_ = reinterpret_cast<uint64_t>(dev);
  c->cap_ = cap;
  return c;
}

U32Cell::~U32Cell() {
  if (host_)
    (void)hipHostFree(host_);
}

// cells.rs:134-149 (TokenIdBuffer::write): the first n slots.
void U32Cell::write(const uint32_t *values, size_t n) {
  if (n > cap_)
    fail("TokenIdBuffer::write: " + std::to_string(n) + " ids exceeds cap " + std::to_string(cap_));
  volatile uint32_t *dst = host_;
  for (size_t i = 0; i < n; ++i)
    dst[i] = values[i];
}

uint32_t U32Cell::read() const { return *static_cast<volatile uint32_t *>(host_); }

} // namespace tensor_ash
