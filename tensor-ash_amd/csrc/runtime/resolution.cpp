// Shape resolution and validation of matmul ops.
// Follows src/matmul/resolution.rs:10-476 rule for rule, with the same
// error text (callers and tests match on substrings of it).
#include <sstream>

#include "internal.hpp"

namespace tensor_ash {

namespace {

std::optional<uint64_t> checked_product(std::initializer_list<uint64_t> values) {
  uint64_t acc = 1;
  for (uint64_t v : values) {
    if (v != 0 && acc > UINT64_MAX / v)
      return std::nullopt;
    acc *= v;
  }
  return acc;
}

} // namespace

std::string fmt_shape(const std::vector<uint32_t> &s) {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < s.size(); ++i)
    o << (i ? ", " : "") << s[i];
  o << "]";
  return o.str();
}

namespace {

void ensure_dim_eq(const char *ll, uint32_t l, const char *rl, uint32_t r) {
  if (l != r) {
    std::ostringstream o;
    o << "matmul shape mismatch: " << ll << "=" << l << " vs " << rl << "=" << r;
    fail(o.str());
  }
}

void ensure_broadcastable(const char *label, uint32_t in, uint32_t out) {
  if (in != 1 && in != out) {
    std::ostringstream o;
    o << "matmul incompatible batch dims: " << label << ".B=" << in
      << " cannot broadcast to C.B=" << out;
    fail(o.str());
  }
}

} // namespace

// resolution.rs:18-44.
MatrixShape MatrixShape::from_tensor_shape(const std::vector<uint32_t> &shape) {
  MatrixShape s{};
  if (shape.size() == 2) {
    s = {1, shape[0], shape[1]};
  } else if (shape.size() == 3) {
    s = {shape[0], shape[1], shape[2]};
  } else {
    fail("tensor rank " + std::to_string(shape.size()) +
         " not supported by matmul (must be 2 or 3)");
  }
  if (s.batch == 0 || s.rows == 0 || s.cols == 0) {
    std::ostringstream o;
    o << "matmul dimensions must be non-zero, got B=" << s.batch << " rows=" << s.rows
      << " cols=" << s.cols;
    fail(o.str());
  }
  return s;
}

// resolution.rs:50-76: batch stride 0 broadcasts; the whole layout must
// be addressable with 32-bit element indices (<= 2^32 elements).
uint32_t MatrixShape::batch_stride(const char *label) const {
  auto plane = checked_product({rows, cols});
  if (!plane)
    fail(std::string(label) + " matrix size overflows u64");
  uint32_t stride = 0;
  if (batch != 1) {
    if (*plane > UINT32_MAX)
      fail(std::string(label) + " batch stride overflows u32");
    stride = (uint32_t)*plane;
  }
  auto elements = checked_product({batch, *plane});
  if (!elements || *elements > (uint64_t)UINT32_MAX + 1) {
    std::ostringstream o;
    o << label << " layout exceeds shader u32 indexing: B=" << batch << " rows=" << rows
      << " cols=" << cols;
    fail(o.str());
  }
  return stride;
}

// resolution.rs:421-441.
ResolvedMatmul ResolvedMatmul::from_shapes(const std::vector<uint32_t> &as,
                                           const std::vector<uint32_t> &bs,
                                           const std::vector<uint32_t> &cs) {
  const MatrixShape a = MatrixShape::from_tensor_shape(as);
  const MatrixShape b = MatrixShape::from_tensor_shape(bs);
  const MatrixShape c = MatrixShape::from_tensor_shape(cs);
  ensure_dim_eq("A.K", a.cols, "B.K", b.rows);
  ensure_dim_eq("A.M", a.rows, "C.M", c.rows);
  ensure_dim_eq("B.N", b.cols, "C.N", c.cols);
  ensure_broadcastable("A", a.batch, c.batch);
  ensure_broadcastable("B", b.batch, c.batch);
  ResolvedMatmul r;
  r.m = a.rows;
  r.n = b.cols;
  r.k = a.cols;
  r.batch = c.batch;
  r.batch_stride_a = a.batch_stride("A");
  r.batch_stride_b = b.batch_stride("B");
  r.batch_stride_c = c.batch_stride("C");
  auto flops = checked_product({2, c.batch, a.rows, b.cols, a.cols});
  if (!flops)
    fail("matmul FLOP count overflows u64");
  r.total_flops = *flops;
  return r;
}

// resolution.rs:124-171.
ResolvedMatmul ResolvedMatmul::from_call(const MatmulCall &call) {
  if (!call.a || !call.b || !call.c)
    fail("matmul call has a null tensor");
  const bool a_f16 = call.a->dtype() == DType::F16;
  if (a_f16) {
    if (call.b->dtype() != DType::F16)
      fail(std::string("matmul with f16 A storage requires f16 B (got ") +
           dtype_name(call.b->dtype()) + ")");
    if (call.c->dtype() != DType::F16)
      fail(std::string("matmul with f16 A storage requires f16 C (got ") +
           dtype_name(call.c->dtype()) + ")");
  } else if (call.c->dtype() != DType::F32) {
    fail(std::string("matmul C must be f32 storage (got ") + dtype_name(call.c->dtype()) + ")");
  }
  ResolvedMatmul r = from_shapes(call.a->shape(), call.b->shape(), call.c->shape());
  r.b_f16 = call.b->dtype() == DType::F16;
  r.a_f16 = a_f16;
  r.packed_b = false;
  if (a_f16 && (r.m % 64 != 0 || r.n % 64 != 0 || r.k % 32 != 0)) {
    std::ostringstream o;
    o << "matmul with f16 A storage routes to the aligned coopmat kernels only: "
         "M/N/K must be multiples of (64, 64, 32), got ("
      << r.m << ", " << r.n << ", " << r.k << ")";
    fail(o.str());
  }
  return r;
}

// resolution.rs:173-212.  The packed decode GEMV here takes M <= 8 rows
// (the reference's packed row kernel takes M == 1 only).
ResolvedMatmul ResolvedMatmul::from_op(const MatmulOp &op) {
  ResolvedMatmul r = from_call(op.call);
  r.packed_b = op.packed_b;
  if (op.packed_b) {
    if (r.m > kGemvMaxRows || r.batch != 1) {
      std::ostringstream o;
      o << "packed-B GEMV requires M <= " << kGemvMaxRows << " and batch == 1 (got M=" << r.m
        << ", batch=" << r.batch << ")";
      fail(o.str());
    }
    if (!r.b_f16)
      fail("packed-B GEMV requires f16 weights");
    if (r.a_f16)
      fail("packed-B GEMV does not support f16 activations");
    if (r.n % 32 != 0)
      fail("packed-B GEMV requires N to be a multiple of 32 (got " + std::to_string(r.n) + ")");
  }
  if (r.a_f16 && (!op.epilogue.is_none() || op.has_decode_fusion()))
    fail("matmul with f16 A storage cannot fuse epilogues, normed-A, or store ops "
         "(the coopmat route has no fused specializations)");
  r.validate_epilogue(op);
  r.validate_normed_a(op);
  r.validate_store(op);
  return r;
}

// resolution.rs:214-241: the normed-A weight rides the bias slot and eps
// the beta slot of the reference's push constants, hence the exclusions
// (kept: they are the op's contract).
void ResolvedMatmul::validate_normed_a(const MatmulOp &op) const {
  if (!op.normed_a)
    return;
  const Tensor *w = op.normed_a->weight;
  if (!w)
    fail("normed-A weight tensor is null");
  if (w->dtype() != DType::F32)
    fail("normed-A weight must be f32 storage");
  if (w->len() != k)
    fail("normed-A weight length " + std::to_string(w->len()) + " must equal K = " +
         std::to_string(k));
  if (op.epilogue.bias)
    fail("normed-A cannot combine with an epilogue bias (both use the bias slot)");
  if (op.epilogue.binary.kind == EpilogueBinary::Kind::AddScaled)
    fail("normed-A cannot combine with the AddScaled epilogue (both use beta)");
}

// resolution.rs:243-316.
void ResolvedMatmul::validate_store(const MatmulOp &op) const {
  if (op.store.is_none())
    return;
  if (m != 1 || batch != 1)
    fail("fused store epilogue requires M == 1 and batch == 1 (got M=" + std::to_string(m) +
         ", batch=" + std::to_string(batch) + ")");
  if (!b_f16)
    fail("fused store epilogue requires f16 weights (f16w row-GEMV routes only)");
  if (op.call.accumulate)
    fail("fused store epilogue cannot combine with accumulate");
  if (!op.epilogue.is_none())
    fail("fused store epilogue cannot combine with a fused epilogue");
  const MatmulStoreDesc &d = op.store.desc;
  if (d.head_dim == 0 || d.head_dim % 2 != 0 || n % d.head_dim != 0)
    fail("store head_dim " + std::to_string(d.head_dim) + " must be even and divide N = " +
         std::to_string(n));
  const bool rope = op.store.kind == MatmulStore::Kind::Rope ||
                    op.store.kind == MatmulStore::Kind::RopeScatter;
  const bool scatter = op.store.kind == MatmulStore::Kind::Scatter ||
                       op.store.kind == MatmulStore::Kind::RopeScatter;
  if (rope) {
    const Tensor *t = op.store.table;
    if (!t)
      fail("store rope table tensor is null");
    if (t->dtype() != DType::F32)
      fail("store rope table must be f32 storage");
    const uint64_t needed = ((uint64_t)d.pos_base + 1) * d.head_dim;
    if (t->len() < needed)
      fail("store rope table len " + std::to_string(t->len()) + " does not cover pos_base " +
           std::to_string(d.pos_base) + " (needs " + std::to_string(needed) + ")");
  }
  if (scatter) {
    const Tensor *dst = op.store.dst;
    if (!dst)
      fail("store destination tensor is null");
    const uint64_t heads = n / d.head_dim;
    const uint64_t last = (uint64_t)d.pos_base * d.pos_scale +
                          (heads - 1) * (uint64_t)d.stride_head +
                          (uint64_t)(d.head_dim - 1) * d.stride_dim;
    if (last >= dst->len())
      fail("store destination access " + std::to_string(last) + " out of bounds for len " +
           std::to_string(dst->len()) + " (pos_base " + std::to_string(d.pos_base) + ", N " +
           std::to_string(n) + ", head_dim " + std::to_string(d.head_dim) + ")");
  }
}

// resolution.rs:318-351.
void ResolvedMatmul::validate_epilogue(const MatmulOp &op) const {
  if (op.epilogue.bias) {
    validate_bias_shape(op.epilogue.bias->shape());
    if (op.epilogue.bias->dtype() != DType::F32)
      fail("epilogue bias must be f32 storage");
  }
  if (op.epilogue.binary.kind != EpilogueBinary::Kind::None && !op.epilogue.binary.d)
    fail("epilogue binary op has no D tensor");
  if (const Tensor *d = op.epilogue.d_tensor()) {
    if (d->shape() != op.call.c->shape())
      fail("epilogue D shape " + fmt_shape(d->shape()) + " must equal C shape " +
           fmt_shape(op.call.c->shape()));
    if (d->dtype() != DType::F32)
      fail("epilogue D operand must be f32 storage");
  }
}

void ResolvedMatmul::validate_bias_shape(const std::vector<uint32_t> &shape) const {
  const std::vector<uint32_t> shared{n}, batched{batch, n};
  if (shape != shared && shape != batched)
    fail("epilogue bias shape " + fmt_shape(shape) + ", expected " + fmt_shape(shared) + " or " +
         fmt_shape(batched));
}

bool ResolvedMatmul::operator==(const ResolvedMatmul &o) const {
  return m == o.m && n == o.n && k == o.k && batch == o.batch &&
         batch_stride_a == o.batch_stride_a && batch_stride_b == o.batch_stride_b &&
         batch_stride_c == o.batch_stride_c && total_flops == o.total_flops &&
         b_f16 == o.b_f16 && a_f16 == o.a_f16 && packed_b == o.packed_b;
}

// resolution.rs:444-449.
uint64_t total_flops(const std::vector<ResolvedMatmul> &resolved) {
  uint64_t acc = 0;
  for (const auto &r : resolved) {
    if (acc > UINT64_MAX - r.total_flops)
      fail("total FLOP count overflows u64");
    acc += r.total_flops;
  }
  return acc;
}

} // namespace tensor_ash
