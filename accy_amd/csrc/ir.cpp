// Program IR, checked type derivation and 16-bit float conversions.
// Checks restate src/tensor/type/dim.zig, src/tensor/type/algebra.zig and src/axis/roles.zig;
// the per-kind derivation restates src/tensor/trace/builder.zig (functions cited inline).
#include "ir.hpp"

#include <cstring>
#include <limits>
#include <sstream>

namespace accy {

size_t dtype_size(DType t) {
  switch (t) {
    case DType::i1: case DType::i8: case DType::u8: return 1;
    case DType::i16: case DType::u16: case DType::f16: case DType::bf16: return 2;
    case DType::i32: case DType::u32: case DType::f32: return 4;
    case DType::i64: case DType::u64: case DType::f64: case DType::key: return 8;
  }
  return 0;
}

const char* dtype_name(DType t) {
  static const char* names[] = {"i1", "i8", "i16", "i32", "i64", "u8", "u16", "u32", "u64",
                                "f16", "bf16", "f32", "f64", "key"};
  unsigned i = (unsigned)t;
  return i < kDTypeCount ? names[i] : "?";
}

bool dtype_is_float(DType t) {
  return t == DType::f16 || t == DType::bf16 || t == DType::f32 || t == DType::f64;
}
bool dtype_is_signed(DType t) {
  return t == DType::i8 || t == DType::i16 || t == DType::i32 || t == DType::i64;
}
bool dtype_is_unsigned(DType t) {
  return t == DType::u8 || t == DType::u16 || t == DType::u32 || t == DType::u64;
}
bool dtype_is_numeric(DType t) { return dtype_is_float(t) || dtype_is_signed(t) || dtype_is_unsigned(t); }

const char* err_name(Err e) {
  static const char* names[] = {
      "Ok", "InvalidArtifact", "BadMagic", "UnsupportedVersion", "UnknownTag", "InvalidReference",
      "TooManyOperands", "ScanTooDeep", "InvalidProgram", "InvalidDimension", "ShapeElementOverflow",
      "ShapeByteOverflow", "ShapeMismatch", "DTypeMismatch", "RankMismatch", "AxisOutOfRange",
      "AxisNotFound", "AxisNameEmpty", "AxisNameReserved", "AxisExtentMismatch", "DuplicateAxis",
      "InvalidPermutation", "ReshapeElementMismatch", "BroadcastRankMismatch",
      "BroadcastDimensionMismatch", "ContractDTypeMismatch", "ReduceInitNotScalar",
      "PayloadLengthMismatch", "InvalidCustomCallContract", "UnsupportedCustomCallArity",
      "ScanLengthNegative", "ScanWithoutCarries", "ScanArityUnsupported", "ScanArityMismatch",
      "ProjectionSourceNotScan", "ProjectionIndexInvalid", "Unsupported"};
  unsigned i = (unsigned)e;
  return i < sizeof(names) / sizeof(names[0]) ? names[i] : "?";
}

void fail(Err c, const std::string& detail) {
  throw Error(c, std::string(err_name(c)) + (detail.empty() ? "" : ": " + detail));
}

const char* kind_name(Kind k) {
  static const char* names[] = {"parameter", "constant", "unary", "binary", "iota", "broadcast",
                                "broadcast_in_dim", "reshape", "transpose", "reduce", "gather",
                                "scatter_add", "sparse_cross_entropy", "dot_general", "compare",
                                "select", "custom_call", "scan", "projection"};
  unsigned i = (unsigned)k;
  return i < kKindCount ? names[i] : "?";
}

int Type::find(const std::string& name) const {
  for (size_t i = 0; i < dims.size(); ++i)
    if (dims[i].name == name) return (int)i;
  return -1;
}

// dimsElementCount (dim.zig:256-266): negative extents are InvalidDimension, usize overflow is
// ShapeElementOverflow.
uint64_t Type::elements() const {
  uint64_t count = 1;
  for (const Dim& d : dims) {
    if (d.extent < 0) fail(Err::InvalidDimension);
    uint64_t e = (uint64_t)d.extent;
    if (e != 0 && count > std::numeric_limits<uint64_t>::max() / e) fail(Err::ShapeElementOverflow);
    count *= e;
  }
  return count;
}

uint64_t Type::bytes() const {
  uint64_t n = elements();
  uint64_t s = dtype_size(dtype);
  if (n != 0 && n > std::numeric_limits<uint64_t>::max() / s) fail(Err::ShapeByteOverflow);
  return n * s;
}

std::string Type::str() const {
  std::ostringstream os;
  os << dtype_name(dtype) << "{";
  for (size_t i = 0; i < dims.size(); ++i) os << (i ? "," : "") << dims[i].name << "=" << dims[i].extent;
  os << "}";
  return os.str();
}

// validateDims (dim.zig:226-233).
void validate_dims(const std::vector<Dim>& dims) {
  for (size_t i = 0; i < dims.size(); ++i) {
    if (dims[i].name.empty()) fail(Err::AxisNameEmpty);
    if (dims[i].extent < 0) fail(Err::InvalidDimension, dims[i].name);
    for (size_t j = 0; j < i; ++j)
      if (dims[j].name == dims[i].name) fail(Err::DuplicateAxis, dims[i].name);
  }
}

// roles.check (src/axis/roles.zig:21-41) over several groups: out of range first, then an axis that
// repeats within or across groups.
static void validate_axis_groups(size_t rank, const std::vector<const std::vector<int64_t>*>& groups) {
  for (size_t g = 0; g < groups.size(); ++g) {
    const auto& group = *groups[g];
    for (size_t a = 0; a < group.size(); ++a) {
      int64_t axis = group[a];
      if (axis < 0 || (uint64_t)axis >= rank) fail(Err::AxisOutOfRange);
      for (size_t p = 0; p < g; ++p)
        for (int64_t seen : *groups[p])
          if (seen == axis) fail(Err::DuplicateAxis);
      for (size_t s = 0; s < a; ++s)
        if (group[s] == axis) fail(Err::DuplicateAxis);
    }
  }
}

void validate_axes(size_t rank, const std::vector<int64_t>& axes) { validate_axis_groups(rank, {&axes}); }

static bool groups_overlap(const std::vector<int64_t>& a, const std::vector<int64_t>& b) {
  for (int64_t x : b)
    for (int64_t y : a)
      if (x == y) return true;
  return false;
}

static bool contains(const std::vector<int64_t>& axes, size_t index) {
  for (int64_t a : axes)
    if (a == (int64_t)index) return true;
  return false;
}

static Type make_type(DType dt, const std::vector<Dim>& dims) {
  validate_dims(dims);
  return Type{dt, dims};
}

static void same_type(const Type& a, const Type& b) {
  if (a.dtype != b.dtype) fail(Err::DTypeMismatch);
  if (!(a.dims == b.dims)) fail(Err::ShapeMismatch, a.str() + " vs " + b.str());
}

// removeAxes (algebra.zig:99-110).
static std::vector<Dim> remove_axes(const std::vector<Dim>& dims, const std::vector<int64_t>& axes) {
  validate_axes(dims.size(), axes);
  std::vector<Dim> out;
  for (size_t i = 0; i < dims.size(); ++i)
    if (!contains(axes, i)) out.push_back(dims[i]);
  return out;
}

// algebra.gather (algebra.zig:482-504).
static Type gather_type(const Type& input, const Type& indices, int64_t axis) {
  if (indices.dtype != DType::i32) fail(Err::DTypeMismatch, "gather indices must be i32");
  validate_axes(input.rank(), {axis});
  std::vector<Dim> dims(input.dims.begin(), input.dims.begin() + axis);
  dims.insert(dims.end(), indices.dims.begin(), indices.dims.end());
  dims.insert(dims.end(), input.dims.begin() + axis + 1, input.dims.end());
  return make_type(input.dtype, dims);
}

Builder::Builder(std::string name) { g_.name = std::move(name); }

void Builder::check(uint32_t id) const {
  if (finished_) fail(Err::InvalidProgram, "builder finished");
  if (id >= g_.ops.size()) fail(Err::InvalidReference);
}

uint32_t Builder::append(Op op) {
  if (finished_) fail(Err::InvalidProgram, "builder finished");
  g_.ops.push_back(std::move(op));
  return (uint32_t)g_.ops.size() - 1;
}

// inputTyped (builder.zig:114-121).
uint32_t Builder::input(const Type& t) {
  Op op;
  op.kind = Kind::parameter;
  op.result = make_type(t.dtype, t.dims);
  op.index = g_.params.size();
  uint32_t id = append(std::move(op));
  g_.params.push_back(id);
  return id;
}

// constantBytes (builder.zig:259-265).
uint32_t Builder::constant(const Type& t, const std::string& payload) {
  Type ty = make_type(t.dtype, t.dims);
  if (payload.size() != ty.bytes()) fail(Err::PayloadLengthMismatch);
  Op op;
  op.kind = Kind::constant;
  op.result = ty;
  op.bytes = payload;
  return append(std::move(op));
}

// iotaTyped (builder.zig:311-314).
uint32_t Builder::iota(const Type& t, int64_t axis) {
  validate_axes(t.rank(), {axis});
  Op op;
  op.kind = Kind::iota;
  op.result = make_type(t.dtype, t.dims);
  op.axis = axis;
  return append(std::move(op));
}

// unary (builder.zig:316-321).
uint32_t Builder::unary(Unary u, uint32_t a) {
  check(a);
  Op op;
  op.kind = Kind::unary;
  op.code = (uint8_t)u;
  op.result = type(a);
  op.args = {a};
  return append(std::move(op));
}

// binary (builder.zig:323-330).
uint32_t Builder::binary(Binary b, uint32_t lhs, uint32_t rhs) {
  check(lhs);
  check(rhs);
  same_type(type(lhs), type(rhs));
  Op op;
  op.kind = Kind::binary;
  op.code = (uint8_t)b;
  op.result = type(lhs);
  op.args = {lhs, rhs};
  return append(std::move(op));
}

// compare (builder.zig:370-378).
uint32_t Builder::compare(Cmp c, uint32_t lhs, uint32_t rhs) {
  check(lhs);
  check(rhs);
  same_type(type(lhs), type(rhs));
  Op op;
  op.kind = Kind::compare;
  op.code = (uint8_t)c;
  op.result = Type{DType::i1, type(lhs).dims};
  op.args = {lhs, rhs};
  return append(std::move(op));
}

// select (builder.zig:395-404; algebra.select at algebra.zig:588-594).
uint32_t Builder::select(uint32_t pred, uint32_t on_true, uint32_t on_false) {
  check(pred);
  check(on_true);
  check(on_false);
  const Type& p = type(pred);
  const Type& t = type(on_true);
  const Type& f = type(on_false);
  if (p.dtype != DType::i1) fail(Err::DTypeMismatch, "select predicate must be i1");
  if (t.dtype != f.dtype) fail(Err::DTypeMismatch);
  if (!(t.dims == f.dims)) fail(Err::ShapeMismatch);
  if (p.rank() != 0 && !(p.dims == t.dims)) fail(Err::ShapeMismatch);
  Op op;
  op.kind = Kind::select;
  op.result = t;
  op.args = {pred, on_true, on_false};
  return append(std::move(op));
}

// broadcastOp (builder.zig:496-506): the result type is taken as given.
uint32_t Builder::broadcast(uint32_t a, const std::vector<Dim>& dims) {
  check(a);
  Op op;
  op.kind = Kind::broadcast;
  op.result = make_type(type(a).dtype, dims);
  op.args = {a};
  for (const Dim& d : dims) op.ints.push_back(d.extent);
  return append(std::move(op));
}

// broadcastTo (builder.zig:508-527; algebra.broadcastInDim at algebra.zig:568-586).
uint32_t Builder::broadcast_in_dim(uint32_t a, const std::vector<Dim>& dims, const std::vector<int64_t>& bdims) {
  check(a);
  const Type& in = type(a);
  if (bdims.size() != in.rank()) fail(Err::BroadcastRankMismatch);
  validate_axes(dims.size(), bdims);
  for (size_t i = 0; i < bdims.size(); ++i) {
    const Dim& target = dims[(size_t)bdims[i]];
    if (in.dims[i].extent != 1 && in.dims[i].extent != target.extent) fail(Err::BroadcastDimensionMismatch);
  }
  Op op;
  op.kind = Kind::broadcast_in_dim;
  op.result = make_type(in.dtype, dims);
  op.args = {a};
  op.ints = bdims;
  return append(std::move(op));
}

// reshapeTo (builder.zig:529-539; algebra.reshaped at algebra.zig:562-566).
uint32_t Builder::reshape(uint32_t a, const std::vector<Dim>& dims) {
  check(a);
  Type ty = make_type(type(a).dtype, dims);
  if (type(a).elements() != ty.elements()) fail(Err::ReshapeElementMismatch);
  Op op;
  op.kind = Kind::reshape;
  op.result = ty;
  op.args = {a};
  for (const Dim& d : dims) op.ints.push_back(d.extent);
  return append(std::move(op));
}

// transposeBy (builder.zig:541-555; algebra.permuted / validatePermutation).
uint32_t Builder::transpose(uint32_t a, const std::vector<int64_t>& perm) {
  check(a);
  const Type& in = type(a);
  if (perm.size() != in.rank()) fail(Err::RankMismatch);
  validate_axes(in.rank(), perm);
  std::vector<Dim> dims;
  for (int64_t p : perm) dims.push_back(in.dims[(size_t)p]);
  Op op;
  op.kind = Kind::transpose;
  op.result = make_type(in.dtype, dims);
  op.args = {a};
  op.ints = perm;
  return append(std::move(op));
}

// reduce (builder.zig:557-579).
uint32_t Builder::reduce(uint32_t a, uint32_t init, Reducer r, const std::vector<int64_t>& dims) {
  check(a);
  check(init);
  if (type(a).dtype != type(init).dtype) fail(Err::DTypeMismatch);
  if (type(init).rank() != 0) fail(Err::ReduceInitNotScalar);
  std::vector<Dim> result = remove_axes(type(a).dims, dims);
  Op op;
  op.kind = Kind::reduce;
  op.code = (uint8_t)r;
  op.result = make_type(type(a).dtype, result);
  op.args = {a, init};
  op.ints = dims;
  return append(std::move(op));
}

// gatherOp (builder.zig:630-646).
uint32_t Builder::gather(uint32_t a, uint32_t indices, int64_t axis) {
  check(a);
  check(indices);
  Op op;
  op.kind = Kind::gather;
  op.result = gather_type(type(a), type(indices), axis);
  op.args = {a, indices};
  op.axis = axis;
  return append(std::move(op));
}

// scatterAddOp (builder.zig:679-704; algebra.scatterAdd at algebra.zig:506-520).
uint32_t Builder::scatter_add(uint32_t a, uint32_t indices, uint32_t updates, int64_t axis) {
  check(a);
  check(indices);
  check(updates);
  const Type& in = type(a);
  if (!dtype_is_numeric(in.dtype)) fail(Err::DTypeMismatch);
  if (type(updates).dtype != in.dtype) fail(Err::DTypeMismatch);
  Type expected = gather_type(in, type(indices), axis);
  if (!(type(updates).dims == expected.dims)) fail(Err::ShapeMismatch);
  Op op;
  op.kind = Kind::scatter_add;
  op.result = in;
  op.args = {a, indices, updates};
  op.axis = axis;
  return append(std::move(op));
}

// sparseCrossEntropyOp (builder.zig:728-741; algebra.sparseCrossEntropy at algebra.zig:522-537).
uint32_t Builder::sparse_cross_entropy(uint32_t logits, uint32_t targets, int64_t axis) {
  check(logits);
  check(targets);
  const Type& l = type(logits);
  const Type& t = type(targets);
  if (!dtype_is_float(l.dtype)) fail(Err::DTypeMismatch);
  if (t.dtype != DType::i32) fail(Err::DTypeMismatch);
  validate_axes(l.rank(), {axis});
  std::vector<Dim> expected = remove_axes(l.dims, {axis});
  if (!(t.dims == expected)) fail(Err::ShapeMismatch);
  Op op;
  op.kind = Kind::sparse_cross_entropy;
  op.result = make_type(l.dtype, t.dims);
  op.args = {logits, targets};
  op.axis = axis;
  return append(std::move(op));
}

// dotGeneralOp (builder.zig:867-897; algebra.dotGeneralDims at algebra.zig:416-480).
uint32_t Builder::dot_general(uint32_t lhs, uint32_t rhs, const std::vector<int64_t>& lc,
                              const std::vector<int64_t>& rc, const std::vector<int64_t>& lb,
                              const std::vector<int64_t>& rb) {
  check(lhs);
  check(rhs);
  const Type& L = type(lhs);
  const Type& R = type(rhs);
  if (L.dtype != R.dtype) fail(Err::ContractDTypeMismatch);
  validate_axes(L.rank(), lc);
  validate_axes(R.rank(), rc);
  validate_axes(L.rank(), lb);
  validate_axes(R.rank(), rb);
  if (groups_overlap(lc, lb)) fail(Err::DuplicateAxis);
  if (groups_overlap(rc, rb)) fail(Err::DuplicateAxis);
  if (lc.size() != rc.size()) fail(Err::RankMismatch);
  if (lb.size() != rb.size()) fail(Err::RankMismatch);
  for (size_t i = 0; i < lc.size(); ++i)
    if (L.dims[(size_t)lc[i]].extent != R.dims[(size_t)rc[i]].extent) fail(Err::AxisExtentMismatch);
  for (size_t i = 0; i < lb.size(); ++i)
    if (L.dims[(size_t)lb[i]].extent != R.dims[(size_t)rb[i]].extent) fail(Err::AxisExtentMismatch);
  std::vector<Dim> dims;
  for (int64_t a : lb) dims.push_back(L.dims[(size_t)a]);
  for (size_t i = 0; i < L.rank(); ++i)
    if (!contains(lc, i) && !contains(lb, i)) dims.push_back(L.dims[i]);
  for (size_t i = 0; i < R.rank(); ++i)
    if (!contains(rc, i) && !contains(rb, i)) dims.push_back(R.dims[i]);
  for (size_t i = 0; i < dims.size(); ++i)
    for (size_t j = 0; j < i; ++j)
      if (dims[j].name == dims[i].name) fail(Err::DuplicateAxis);
  Op op;
  op.kind = Kind::dot_general;
  op.result = make_type(L.dtype, dims);
  op.args = {lhs, rhs};
  op.lhs_contract = lc;
  op.rhs_contract = rc;
  op.lhs_batch = lb;
  op.rhs_batch = rb;
  return append(std::move(op));
}

// customCall (builder.zig:343-368).
uint32_t Builder::custom_call(const std::string& target, uint32_t version, const std::vector<uint32_t>& operands,
                              const Type& result) {
  if (target.empty()) fail(Err::InvalidCustomCallContract);
  if (version == 0) fail(Err::InvalidCustomCallContract);
  if (operands.size() > kMaxCustomCallOperands) fail(Err::UnsupportedCustomCallArity);
  for (uint32_t a : operands) check(a);
  Op op;
  op.kind = Kind::custom_call;
  op.result = make_type(result.dtype, result.dims);
  op.args = operands;
  op.bytes = target;
  op.index = version;
  return append(std::move(op));
}

// emitScanIds (builder.zig:964-990).
uint32_t Builder::scan(int64_t length, const std::vector<uint32_t>& inits, std::shared_ptr<const Graph> body) {
  if (length < 0) fail(Err::ScanLengthNegative);
  if (inits.empty()) fail(Err::ScanWithoutCarries);
  if (inits.size() > kMaxScanCarries) fail(Err::ScanArityUnsupported);
  if (body->params.size() != inits.size()) fail(Err::ScanArityMismatch);
  if (body->outputs.size() != inits.size()) fail(Err::ScanArityMismatch);
  for (size_t i = 0; i < inits.size(); ++i) {
    check(inits[i]);
    same_type(type(inits[i]), body->type(body->params[i]));
    same_type(type(inits[i]), body->type(body->outputs[i]));
  }
  Op op;
  op.kind = Kind::scan;
  op.result = type(inits[0]);
  op.args = inits;
  op.axis = length;
  op.body = std::move(body);
  return append(std::move(op));
}

// projection (builder.zig:941-951).
uint32_t Builder::projection(uint32_t source, uint64_t index) {
  check(source);
  const Op& src = g_.ops[source];
  if (src.kind != Kind::scan) fail(Err::ProjectionSourceNotScan);
  if (index == 0 || index >= src.args.size()) fail(Err::ProjectionIndexInvalid);
  Op op;
  op.kind = Kind::projection;
  op.result = src.body->type(src.body->outputs[index]);
  op.args = {source};
  op.index = index;
  return append(std::move(op));
}

// finish (builder.zig:992-1008).
Graph Builder::finish(const std::vector<uint32_t>& outputs) {
  if (finished_) fail(Err::InvalidProgram, "builder finished");
  for (uint32_t o : outputs) check(o);
  finished_ = true;
  Graph g = std::move(g_);
  g.outputs = outputs;
  return g;
}

std::vector<int64_t> row_major_strides(const std::vector<Dim>& dims) {
  std::vector<int64_t> s(dims.size(), 1);
  for (int i = (int)dims.size() - 2; i >= 0; --i) s[i] = s[i + 1] * dims[i + 1].extent;
  return s;
}

// A constant whose payload repeats one element (the splat constants the tracer's `full` writes).
bool is_splat_constant(const Op& op) {
  if (op.kind != Kind::constant) return false;
  size_t es = dtype_size(op.result.dtype);
  if (op.bytes.size() < es) return false;
  for (size_t off = es; off + es <= op.bytes.size(); off += es)
    if (std::memcmp(op.bytes.data(), op.bytes.data() + off, es) != 0) return false;
  return true;
}

// IEEE binary16 conversion, round to nearest even, with subnormals, infinities and NaN.
uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) {
    if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
    return (uint16_t)(sign | 0x7c00u);
  }
  int32_t e = (int32_t)exp - 127 + 15;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t m = man | 0x800000u;
    uint32_t shift = (uint32_t)(14 - e);
    uint32_t half = 1u << (shift - 1);
    uint32_t rem = m & ((1u << shift) - 1);
    uint32_t out = m >> shift;
    if (rem > half || (rem == half && (out & 1u))) out += 1;
    return (uint16_t)(sign | out);
  }
  uint32_t out = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) out += 1;  // may carry into the exponent
  return (uint16_t)(sign | out);
}

float f16_bits_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t x;
  if (exp == 0) {
    if (man == 0) {
      x = sign;
    } else {
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while (!(man & 0x400u));
      x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 0x1f) {
    x = sign | 0x7f800000u | (man << 13);
  } else {
    x = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

uint16_t f32_to_bf16_trunc(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  return (uint16_t)(x >> 16);
}

float bf16_bits_to_f32(uint16_t h) {
  uint32_t x = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

}  // namespace accy
