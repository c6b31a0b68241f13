// Tensor program IR for the HIP execution target.
//
// Mirrors the reference's program model: element types (deps/lib/compiler/gpu/abi/src/dtype.zig:37-51),
// named dimensions and types (src/tensor/type/dim.zig:62-146), operation kinds and their payloads
// (src/tensor/program.zig:14-282). A Builder appends one operation at a time and derives every result
// type itself with the same checks and error names as the reference tracer's `Builder.operation`
// (src/tensor/trace/builder.zig:123-179; src/tensor/type/algebra.zig:10-200), which is what lets the
// wire decoder refuse bytes that carry a wrong type.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace accy {

enum class DType : uint8_t { i1 = 0, i8, i16, i32, i64, u8, u16, u32, u64, f16, bf16, f32, f64, key };
constexpr int kDTypeCount = 14;

size_t dtype_size(DType t);
const char* dtype_name(DType t);
bool dtype_is_float(DType t);
bool dtype_is_signed(DType t);
bool dtype_is_unsigned(DType t);
bool dtype_is_numeric(DType t);

struct Dim {
  std::string name;
  int64_t extent = 0;
  bool operator==(const Dim& o) const { return extent == o.extent && name == o.name; }
};

// Failure names follow the reference's error sets: wire (src/tensor/wire/format.zig:36-43), shape
// algebra (src/tensor/type/dim.zig:8-30) and the builder's own checks (builder.zig).
enum class Err : uint8_t {
  Ok = 0,
  InvalidArtifact,
  BadMagic,
  UnsupportedVersion,
  UnknownTag,
  InvalidReference,
  TooManyOperands,
  ScanTooDeep,
  InvalidProgram,
  InvalidDimension,
  ShapeElementOverflow,
  ShapeByteOverflow,
  ShapeMismatch,
  DTypeMismatch,
  RankMismatch,
  AxisOutOfRange,
  AxisNotFound,
  AxisNameEmpty,
  AxisNameReserved,
  AxisExtentMismatch,
  DuplicateAxis,
  InvalidPermutation,
  ReshapeElementMismatch,
  BroadcastRankMismatch,
  BroadcastDimensionMismatch,
  ContractDTypeMismatch,
  ReduceInitNotScalar,
  PayloadLengthMismatch,
  InvalidCustomCallContract,
  UnsupportedCustomCallArity,
  ScanLengthNegative,
  ScanWithoutCarries,
  ScanArityUnsupported,
  ScanArityMismatch,
  ProjectionSourceNotScan,
  ProjectionIndexInvalid,
  Unsupported,
};
const char* err_name(Err e);

struct Error : std::runtime_error {
  Err code;
  Error(Err c, const std::string& detail) : std::runtime_error(detail), code(c) {}
};
[[noreturn]] void fail(Err c, const std::string& detail = "");

struct Type {
  DType dtype = DType::f32;
  std::vector<Dim> dims;
  size_t rank() const { return dims.size(); }
  int find(const std::string& name) const;
  uint64_t elements() const;  // throws ShapeElementOverflow / InvalidDimension
  uint64_t bytes() const;     // throws ShapeByteOverflow
  bool operator==(const Type& o) const { return dtype == o.dtype && dims == o.dims; }
  std::string str() const;
};

enum class Kind : uint8_t {
  parameter = 0,
  constant,
  unary,
  binary,
  iota,
  broadcast,
  broadcast_in_dim,
  reshape,
  transpose,
  reduce,
  gather,
  scatter_add,
  sparse_cross_entropy,
  dot_general,
  compare,
  select,
  custom_call,
  scan,
  projection,
};
constexpr int kKindCount = 19;
const char* kind_name(Kind k);

enum class Unary : uint8_t { neg = 0, abs, exp, log, sqrt, tanh, sin, cos, tan };
enum class Binary : uint8_t { add = 0, sub, mul, div, max, min, pow };
enum class Reducer : uint8_t { sum = 0, max, min };
enum class Cmp : uint8_t { lt = 0, le, gt, ge, eq, ne };
constexpr int kUnaryCount = 9, kBinaryCount = 7, kReducerCount = 3, kCmpCount = 6;

// Operand and payload bounds from src/tensor/program.zig:144-146.
constexpr size_t kMaxCustomCallOperands = 4;
constexpr size_t kMaxOperationOperands = 8;
constexpr size_t kMaxScanCarries = 8;

struct Graph;

struct Op {
  Kind kind = Kind::parameter;
  Type result;
  uint8_t code = 0;            // Unary / Binary / Reducer / Cmp code
  std::vector<uint32_t> args;  // operand ids in the order the reference lists them
  std::vector<int64_t> ints;   // broadcast_dims, permutation, reduce dimensions, sizes / new_shape
  std::vector<int64_t> lhs_contract, rhs_contract, lhs_batch, rhs_batch;
  int64_t axis = 0;            // iota / gather / scatter_add / sparse_cross_entropy axis; scan length
  uint64_t index = 0;          // parameter index, projection index, custom_call version
  std::string bytes;           // constant payload or custom_call target
  std::shared_ptr<const Graph> body;  // scan body
};

struct Graph {
  std::string name;
  std::vector<Op> ops;
  std::vector<uint32_t> params;
  std::vector<uint32_t> outputs;
  const Type& type(uint32_t id) const { return ops.at(id).result; }
};
using Program = Graph;

// Dims checks from src/tensor/type/dim.zig:217-241.
void validate_dims(const std::vector<Dim>& dims);
void validate_axes(size_t rank, const std::vector<int64_t>& axes);

// Appends operations one at a time and derives every result type (src/tensor/trace/builder.zig).
class Builder {
 public:
  explicit Builder(std::string name);
  uint32_t size() const { return (uint32_t)g_.ops.size(); }
  const Type& type(uint32_t id) const { return g_.ops.at(id).result; }
  const Op& op(uint32_t id) const { return g_.ops.at(id); }

  uint32_t input(const Type& t);
  uint32_t constant(const Type& t, const std::string& payload);
  uint32_t iota(const Type& t, int64_t axis);
  uint32_t unary(Unary u, uint32_t a);
  uint32_t binary(Binary b, uint32_t lhs, uint32_t rhs);
  uint32_t compare(Cmp c, uint32_t lhs, uint32_t rhs);
  uint32_t select(uint32_t pred, uint32_t on_true, uint32_t on_false);
  uint32_t broadcast(uint32_t a, const std::vector<Dim>& dims);
  uint32_t broadcast_in_dim(uint32_t a, const std::vector<Dim>& dims, const std::vector<int64_t>& bdims);
  uint32_t reshape(uint32_t a, const std::vector<Dim>& dims);
  uint32_t transpose(uint32_t a, const std::vector<int64_t>& perm);
  uint32_t reduce(uint32_t a, uint32_t init, Reducer r, const std::vector<int64_t>& dims);
  uint32_t gather(uint32_t a, uint32_t indices, int64_t axis);
  uint32_t scatter_add(uint32_t a, uint32_t indices, uint32_t updates, int64_t axis);
  uint32_t sparse_cross_entropy(uint32_t logits, uint32_t targets, int64_t axis);
  uint32_t dot_general(uint32_t lhs, uint32_t rhs, const std::vector<int64_t>& lc, const std::vector<int64_t>& rc,
                       const std::vector<int64_t>& lb, const std::vector<int64_t>& rb);
  uint32_t custom_call(const std::string& target, uint32_t version, const std::vector<uint32_t>& operands,
                       const Type& result);
  uint32_t scan(int64_t length, const std::vector<uint32_t>& inits, std::shared_ptr<const Graph> body);
  uint32_t projection(uint32_t source, uint64_t index);

  Graph finish(const std::vector<uint32_t>& outputs);

 private:
  uint32_t append(Op op);
  void check(uint32_t id) const;
  Graph g_;
  bool finished_ = false;
};

// ---- evaluation helpers shared by planners and evaluators ----
std::vector<int64_t> row_major_strides(const std::vector<Dim>& dims);
bool is_splat_constant(const Op& op);
uint16_t f32_to_f16_bits(float f);  // round to nearest even
float f16_bits_to_f32(uint16_t h);
uint16_t f32_to_bf16_trunc(float f);  // Bf16.fromF32 (constants and operation results), dtype.zig:6-9
float bf16_bits_to_f32(uint16_t h);

}  // namespace accy
