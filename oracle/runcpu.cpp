// ORACLE — test infrastructure only. A CPU restatement of the reference's `tensor.runCpu` semantics,
// used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker for the HIP
// target. Nothing in the accy_amd product loads, links or calls this file.
//
// The program is decoded from ACTP v1 wire bytes with the shared codec (accy_amd/csrc/wire.cpp) and
// evaluated one operation at a time with the reference's arithmetic rules:
//  * reductions: out[o] = fold(init, x[o, r]) left to right over r, one output at a time, with an f32
//    accumulator for 16-bit inputs rounded once at the store
//    (src/preparation/kernelization/lowering/reduction.zig:839-878, 1157-1177);
//  * dot_general: per output a serial f32 `acc = acc + a*b` over the contracted index, multiply and
//    add rounded separately (lowering/dot.zig:2049-2115; choir x64 scalar.zig:925-962 emits FMA only
//    for an explicit fma op) — this file is built with -ffp-contract=off;
//  * 16-bit floats compute in f32 and round back after every operation (src/eval/root.zig:14-16):
//    f16 to nearest even (Zig @floatCast), bf16 by truncation (Bf16.fromF32 keeps the high 16 bits,
//    deps/lib/compiler/gpu/abi/src/dtype.zig:6-9; used for every bf16 result of the evaluator,
//    src/eval/evaluator.zig:2242-2244 binary, 2338 unary, 2384-2386 pow, 2860 convert), so
//    reductions and dots that accumulate bf16 in f32 also truncate at the store;
//  * sin/cos/tan/exp/log/tanh/pow are libm calls (deps/lib/base/sys/src/math.zig:58-125;
//    scalar.zig:804-828), sqrt is the correctly rounded sqrt (scalar.zig:736);
//  * gather clamps indices into [0, extent-1] (lowering/elementwise.zig:1190-1208);
//  * integer add/sub/mul wrap, integer division truncates and division by zero is an error
//    (src/eval/root.zig:11-13).
// Parity pinning: see tests/test_oracle.py (closed forms, the reference README / example known
// answers, f64 brute force, numpy float16 rounding). The exact bits of Zig's @sin/@exp/@log and
// std.math.tanh/pow are not pinned: those live in the Zig toolchain, which is not available.
#include <omp.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <limits>
#include <map>
#include <string>
#include <vector>

#include "../accy_amd/csrc/ir.hpp"
#include "../accy_amd/csrc/wire.hpp"

using namespace accy;

namespace {

struct Tensor {
  Type type;
  std::vector<uint8_t> data;
  uint64_t n() const { return type.elements(); }
  template <class T> T* as() { return reinterpret_cast<T*>(data.data()); }
  template <class T> const T* as() const { return reinterpret_cast<const T*>(data.data()); }
};

thread_local std::string g_error;

// ---- element access in the compute domain: double for floats (exactly representing f32/f16/bf16),
// with results rounded back to the storage format after every operation. ----
inline double load_f(const Tensor& t, uint64_t i) {
  switch (t.type.dtype) {
    case DType::f16: return f16_bits_to_f32(t.as<uint16_t>()[i]);
    case DType::bf16: return bf16_bits_to_f32(t.as<uint16_t>()[i]);
    case DType::f32: return t.as<float>()[i];
    case DType::f64: return t.as<double>()[i];
    default: fail(Err::Unsupported, "not a float tensor");
  }
}

inline int64_t load_i(const Tensor& t, uint64_t i) {
  switch (t.type.dtype) {
    case DType::i1: return t.as<uint8_t>()[i] ? 1 : 0;
    case DType::i8: return t.as<int8_t>()[i];
    case DType::i16: return t.as<int16_t>()[i];
    case DType::i32: return t.as<int32_t>()[i];
    case DType::i64: return t.as<int64_t>()[i];
    case DType::u8: return t.as<uint8_t>()[i];
    case DType::u16: return t.as<uint16_t>()[i];
    case DType::u32: return t.as<uint32_t>()[i];
    case DType::u64: case DType::key: return (int64_t)t.as<uint64_t>()[i];
    default: fail(Err::Unsupported, "not an integer tensor");
  }
}

inline void store_i(Tensor& t, uint64_t i, int64_t v) {
  switch (t.type.dtype) {
    case DType::i1: t.as<uint8_t>()[i] = v ? 1 : 0; break;
    case DType::i8: t.as<int8_t>()[i] = (int8_t)v; break;
    case DType::i16: t.as<int16_t>()[i] = (int16_t)v; break;
    case DType::i32: t.as<int32_t>()[i] = (int32_t)v; break;
    case DType::i64: t.as<int64_t>()[i] = v; break;
    case DType::u8: t.as<uint8_t>()[i] = (uint8_t)v; break;
    case DType::u16: t.as<uint16_t>()[i] = (uint16_t)v; break;
    case DType::u32: t.as<uint32_t>()[i] = (uint32_t)v; break;
    case DType::u64: case DType::key: t.as<uint64_t>()[i] = (uint64_t)v; break;
    default: fail(Err::Unsupported);
  }
}

// Rounds a value computed in f32 (or f64 for f64 tensors) into the storage format: f16 to nearest
// even (@floatCast), bf16 by truncation (Bf16.fromF32, dtype.zig:6-9; evaluator.zig:2242-2244).
inline void store_f(Tensor& t, uint64_t i, double v) {
  switch (t.type.dtype) {
    case DType::f16: t.as<uint16_t>()[i] = f32_to_f16_bits((float)v); break;
    case DType::bf16: t.as<uint16_t>()[i] = f32_to_bf16_trunc((float)v); break;
    case DType::f32: t.as<float>()[i] = (float)v; break;
    case DType::f64: t.as<double>()[i] = v; break;
    default: fail(Err::Unsupported);
  }
}

Tensor make(const Type& t) {
  Tensor r;
  r.type = t;
  r.data.assign(t.bytes(), 0);
  return r;
}

bool is_f32_domain(DType d) { return d == DType::f16 || d == DType::bf16 || d == DType::f32; }

float unary_f32(Unary u, float x) {
  switch (u) {
    case Unary::neg: return -x;
    case Unary::abs: return std::fabs(x);
    case Unary::exp: return expf(x);
    case Unary::log: return logf(x);
    case Unary::sqrt: return sqrtf(x);
    case Unary::tanh: return tanhf(x);
    case Unary::sin: return sinf(x);
    case Unary::cos: return cosf(x);
    case Unary::tan: return tanf(x);
  }
  return x;
}

double unary_f64(Unary u, double x) {
  switch (u) {
    case Unary::neg: return -x;
    case Unary::abs: return std::fabs(x);
    case Unary::exp: return std::exp(x);
    case Unary::log: return std::log(x);
    case Unary::sqrt: return std::sqrt(x);
    case Unary::tanh: return std::tanh(x);
    case Unary::sin: return std::sin(x);
    case Unary::cos: return std::cos(x);
    case Unary::tan: return std::tan(x);
  }
  return x;
}

// Float max / min as the reference's x64 backend emits them
// (deps/lib/compiler/choir/src/backends/x64/scalar.zig:675-720): maxss / minss, which return the
// second operand on a tie and when either operand is NaN, then the first operand when that result is
// NaN. NaN is thus skipped unless both are NaN, and a +0 / -0 tie gives the second operand.
template <typename F> F ref_max(F a, F b) {
  const F r = a > b ? a : b;
  return r != r ? a : r;
}
template <typename F> F ref_min(F a, F b) {
  const F r = a < b ? a : b;
  return r != r ? a : r;
}

float binary_f32(Binary b, float x, float y) {
  switch (b) {
    case Binary::add: return x + y;
    case Binary::sub: return x - y;
    case Binary::mul: return x * y;
    case Binary::div: return x / y;
    case Binary::max: return ref_max(x, y);
    case Binary::min: return ref_min(x, y);
    case Binary::pow: return powf(x, y);
  }
  return x;
}

double binary_f64(Binary b, double x, double y) {
  switch (b) {
    case Binary::add: return x + y;
    case Binary::sub: return x - y;
    case Binary::mul: return x * y;
    case Binary::div: return x / y;
    case Binary::max: return ref_max(x, y);
    case Binary::min: return ref_min(x, y);
    case Binary::pow: return std::pow(x, y);
  }
  return x;
}

// Integer arithmetic wraps at the declared width (stores truncate); division truncates toward zero.
int64_t binary_int(Binary b, int64_t x, int64_t y, bool is_unsigned) {
  uint64_t ux = (uint64_t)x, uy = (uint64_t)y;
  switch (b) {
    case Binary::add: return (int64_t)(ux + uy);
    case Binary::sub: return (int64_t)(ux - uy);
    case Binary::mul: return (int64_t)(ux * uy);
    case Binary::div:
      if (y == 0) fail(Err::Unsupported, "integer division by zero");
      if (is_unsigned) return (int64_t)(ux / uy);
      if (x == INT64_MIN && y == -1) return x;
      return x / y;
    case Binary::max: return is_unsigned ? (int64_t)(ux > uy ? ux : uy) : (x > y ? x : y);
    case Binary::min: return is_unsigned ? (int64_t)(ux < uy ? ux : uy) : (x < y ? x : y);
    case Binary::pow: fail(Err::Unsupported, "integer pow");
  }
  return x;
}

// Strided gather over the output's row-major index space: out[i] = in[sum(coord_d * stride_d)].
void strided_copy(const Tensor& in, Tensor& out, const std::vector<int64_t>& in_stride_per_out_dim) {
  const auto& od = out.type.dims;
  size_t rank = od.size();
  uint64_t n = out.n();
  size_t es = dtype_size(out.type.dtype);
  if (n == 0) return;
  if (rank == 0) {
    std::memcpy(out.data.data(), in.data.data(), es);
    return;
  }
  int64_t inner = od[rank - 1].extent;
  uint64_t outer = inner ? n / (uint64_t)inner : 0;
  int64_t inner_stride = in_stride_per_out_dim[rank - 1];
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < (int64_t)outer; ++o) {
    int64_t rem = o, base = 0;
    for (int d = (int)rank - 2; d >= 0; --d) {
      int64_t c = rem % od[d].extent;
      rem /= od[d].extent;
      base += c * in_stride_per_out_dim[d];
    }
    const uint8_t* src = in.data.data();
    uint8_t* dst = out.data.data() + (uint64_t)o * inner * es;
    for (int64_t j = 0; j < inner; ++j) std::memcpy(dst + j * es, src + (base + j * inner_stride) * es, es);
  }
}

class Evaluator {
 public:
  explicit Evaluator(const Graph& g) : g_(g) {}

  std::vector<Tensor> run(std::vector<Tensor> inputs) {
    std::vector<Tensor> vals(g_.ops.size());
    std::vector<int> uses(g_.ops.size(), 0);
    for (const Op& op : g_.ops)
      for (uint32_t a : op.args) uses[a]++;
    for (uint32_t o : g_.outputs) uses[o] += 1 << 20;
    for (size_t i = 0; i < g_.ops.size(); ++i) {
      const Op& op = g_.ops[i];
      vals[i] = eval(op, vals, inputs);
      for (uint32_t a : op.args)
        if (--uses[a] == 0) std::vector<uint8_t>().swap(vals[a].data);
    }
    std::vector<Tensor> outs;
    for (uint32_t o : g_.outputs) outs.push_back(vals[o]);
    return outs;
  }

 private:
  const Graph& g_;

  Tensor eval(const Op& op, std::vector<Tensor>& v, std::vector<Tensor>& inputs) {
    const Type& rt = op.result;
    switch (op.kind) {
      case Kind::parameter: return inputs.at(op.index);
      case Kind::constant: {
        Tensor t = make(rt);
        std::memcpy(t.data.data(), op.bytes.data(), op.bytes.size());
        return t;
      }
      case Kind::iota: {
        Tensor t = make(rt);
        auto strides = row_major_strides(rt.dims);
        int64_t ext = rt.dims[(size_t)op.axis].extent, st = strides[(size_t)op.axis];
        uint64_t n = t.n();
        for (uint64_t i = 0; i < n; ++i) {
          int64_t c = ((int64_t)i / st) % ext;
          if (dtype_is_float(rt.dtype)) store_f(t, i, (double)c);
          else store_i(t, i, c);
        }
        return t;
      }
      case Kind::unary: return unary(op, v[op.args[0]]);
      case Kind::binary: return binary(op, v[op.args[0]], v[op.args[1]]);
      case Kind::compare: return compare(op, v[op.args[0]], v[op.args[1]]);
      case Kind::select: return select(op, v[op.args[0]], v[op.args[1]], v[op.args[2]]);
      case Kind::broadcast_in_dim: {
        const Tensor& in = v[op.args[0]];
        Tensor t = make(rt);
        auto is = row_major_strides(in.type.dims);
        std::vector<int64_t> s(rt.rank(), 0);
        for (size_t j = 0; j < op.ints.size(); ++j)
          if (in.type.dims[j].extent != 1) s[(size_t)op.ints[j]] = is[j];
        strided_copy(in, t, s);
        return t;
      }
      case Kind::broadcast: {
        // The reference lowers `broadcast` only from a splat (lowering/elementwise.zig:943-957):
        // a one-element input fills the result; an input of equal size is copied as is.
        const Tensor& in = v[op.args[0]];
        Tensor t = make(rt);
        size_t es = dtype_size(rt.dtype);
        if (in.n() == 1) {
          for (uint64_t i = 0; i < t.n(); ++i) std::memcpy(t.data.data() + i * es, in.data.data(), es);
        } else if (in.n() == t.n()) {
          t.data = in.data;
        } else {
          fail(Err::Unsupported, "broadcast of a non-splat operand");
        }
        return t;
      }
      case Kind::reshape: {
        Tensor t;
        t.type = rt;
        t.data = v[op.args[0]].data;
        return t;
      }
      case Kind::transpose: {
        const Tensor& in = v[op.args[0]];
        Tensor t = make(rt);
        auto is = row_major_strides(in.type.dims);
        std::vector<int64_t> s(rt.rank());
        for (size_t d = 0; d < rt.rank(); ++d) s[d] = is[(size_t)op.ints[d]];
        strided_copy(in, t, s);
        return t;
      }
      case Kind::reduce: return reduce(op, v[op.args[0]], v[op.args[1]]);
      case Kind::dot_general: return dot(op, v[op.args[0]], v[op.args[1]]);
      case Kind::gather: return gather(op, v[op.args[0]], v[op.args[1]]);
      case Kind::scatter_add: return scatter_add(op, v[op.args[0]], v[op.args[1]], v[op.args[2]]);
      case Kind::scan: {
        std::vector<Tensor> carries;
        for (uint32_t a : op.args) carries.push_back(v[a]);
        for (int64_t s = 0; s < op.axis; ++s) carries = Evaluator(*op.body).run(carries);
        scans_[&op] = carries;
        return carries[0];
      }
      case Kind::projection: {
        const Op& src = g_.ops[op.args[0]];
        return scans_.at(&src).at(op.index);
      }
      case Kind::sparse_cross_entropy: return sparse_cross_entropy(op, v[op.args[0]], v[op.args[1]]);
      case Kind::custom_call: fail(Err::Unsupported, "custom_call " + op.bytes);
    }
    fail(Err::Unsupported);
  }

  std::map<const Op*, std::vector<Tensor>> scans_;

  // runCpu takes the expanded form (src/tensor/lower.zig:914-1003; no kernel library is configured,
  // lower.zig:178-182): the op sequence is rebuilt here with the checked builder and evaluated with
  // this file's own reduce / elementwise rules. m starts from the lowest finite value
  // (lower.zig:1005-1029), so a row of -inf keeps m finite.
  Tensor sparse_cross_entropy(const Op& op, const Tensor& logits, const Tensor& targets) {
    const Type& lt = logits.type;
    const DType dt = lt.dtype;
    std::string lowest(dtype_size(dt), '\0');
    if (dt == DType::f16) {
      const uint16_t h = f32_to_f16_bits(-65504.0f);
      std::memcpy(&lowest[0], &h, 2);
    } else if (dt == DType::bf16) {
      const uint16_t h = f32_to_bf16_trunc(-std::numeric_limits<float>::max());
      std::memcpy(&lowest[0], &h, 2);
    } else if (dt == DType::f32) {
      const float f = -std::numeric_limits<float>::max();
      std::memcpy(&lowest[0], &f, 4);
    } else {
      const double d = -std::numeric_limits<double>::max();
      std::memcpy(&lowest[0], &d, 8);
    }
    Builder b("sparse_cross_entropy");
    const uint32_t x = b.input(lt), t = b.input(targets.type);
    std::vector<int64_t> rest;
    for (int64_t d = 0; d < (int64_t)lt.rank(); ++d)
      if (d != op.axis) rest.push_back(d);
    const uint32_t lo = b.constant(Type{dt, {}}, lowest);
    const uint32_t zero = b.constant(Type{dt, {}}, std::string(dtype_size(dt), '\0'));
    const uint32_t row_max = b.reduce(x, lo, Reducer::max, {op.axis});
    const uint32_t shifted = b.binary(Binary::sub, x, b.broadcast_in_dim(row_max, lt.dims, rest));
    const uint32_t denominator = b.reduce(b.unary(Unary::exp, shifted), zero, Reducer::sum, {op.axis});
    const uint32_t positions = b.iota(Type{DType::i32, lt.dims}, op.axis);
    const uint32_t wanted = b.broadcast_in_dim(t, lt.dims, rest);
    const uint32_t on_target = b.compare(Cmp::eq, positions, wanted);
    const uint32_t kept = b.select(on_target, shifted, b.broadcast_in_dim(zero, lt.dims, {}));
    const uint32_t target_shifted = b.reduce(kept, zero, Reducer::sum, {op.axis});
    const uint32_t loss = b.binary(Binary::sub, b.unary(Unary::log, denominator), target_shifted);
    const Graph g = b.finish({loss});
    return Evaluator(g).run({logits, targets})[0];
  }

  Tensor unary(const Op& op, const Tensor& a) {
    Tensor t = make(op.result);
    uint64_t n = t.n();
    Unary u = (Unary)op.code;
    DType d = op.result.dtype;
    if (d == DType::f32) {
      const float* x = a.as<float>();
      float* y = t.as<float>();
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < (int64_t)n; ++i) y[i] = unary_f32(u, x[i]);
    } else if (is_f32_domain(d)) {
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < (int64_t)n; ++i) store_f(t, i, unary_f32(u, (float)load_f(a, i)));
    } else if (d == DType::f64) {
      for (uint64_t i = 0; i < n; ++i) store_f(t, i, unary_f64(u, load_f(a, i)));
    } else {
      bool uns = dtype_is_unsigned(d);
      for (uint64_t i = 0; i < n; ++i) {
        int64_t x = load_i(a, i);
        if (u == Unary::neg) store_i(t, i, (int64_t)(0 - (uint64_t)x));
        else if (u == Unary::abs) store_i(t, i, uns ? x : (x < 0 ? (int64_t)(0 - (uint64_t)x) : x));
        else fail(Err::Unsupported, "transcendental on integers");
      }
    }
    return t;
  }

  Tensor binary(const Op& op, const Tensor& a, const Tensor& b) {
    Tensor t = make(op.result);
    uint64_t n = t.n();
    Binary o = (Binary)op.code;
    DType d = op.result.dtype;
    if (d == DType::f32) {
      const float* x = a.as<float>();
      const float* y = b.as<float>();
      float* z = t.as<float>();
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < (int64_t)n; ++i) z[i] = binary_f32(o, x[i], y[i]);
    } else if (is_f32_domain(d)) {
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < (int64_t)n; ++i)
        store_f(t, i, binary_f32(o, (float)load_f(a, i), (float)load_f(b, i)));
    } else if (d == DType::f64) {
      for (uint64_t i = 0; i < n; ++i) store_f(t, i, binary_f64(o, load_f(a, i), load_f(b, i)));
    } else {
      bool uns = dtype_is_unsigned(d) || d == DType::key;
      for (uint64_t i = 0; i < n; ++i) store_i(t, i, binary_int(o, load_i(a, i), load_i(b, i), uns));
    }
    return t;
  }

  Tensor compare(const Op& op, const Tensor& a, const Tensor& b) {
    Tensor t = make(op.result);
    uint64_t n = t.n();
    Cmp c = (Cmp)op.code;
    DType d = a.type.dtype;
    bool fl = dtype_is_float(d), uns = dtype_is_unsigned(d) || d == DType::key;
    for (uint64_t i = 0; i < n; ++i) {
      bool r;
      if (fl) {
        double x = load_f(a, i), y = load_f(b, i);
        switch (c) {
          case Cmp::lt: r = x < y; break;
          case Cmp::le: r = x <= y; break;
          case Cmp::gt: r = x > y; break;
          case Cmp::ge: r = x >= y; break;
          case Cmp::eq: r = x == y; break;
          default: r = x != y; break;
        }
      } else if (uns) {
        uint64_t x = (uint64_t)load_i(a, i), y = (uint64_t)load_i(b, i);
        switch (c) {
          case Cmp::lt: r = x < y; break;
          case Cmp::le: r = x <= y; break;
          case Cmp::gt: r = x > y; break;
          case Cmp::ge: r = x >= y; break;
          case Cmp::eq: r = x == y; break;
          default: r = x != y; break;
        }
      } else {
        int64_t x = load_i(a, i), y = load_i(b, i);
        switch (c) {
          case Cmp::lt: r = x < y; break;
          case Cmp::le: r = x <= y; break;
          case Cmp::gt: r = x > y; break;
          case Cmp::ge: r = x >= y; break;
          case Cmp::eq: r = x == y; break;
          default: r = x != y; break;
        }
      }
      t.as<uint8_t>()[i] = r ? 1 : 0;
    }
    return t;
  }

  Tensor select(const Op& op, const Tensor& p, const Tensor& a, const Tensor& b) {
    Tensor t = make(op.result);
    uint64_t n = t.n();
    size_t es = dtype_size(op.result.dtype);
    bool scalar_pred = p.type.rank() == 0;
    for (uint64_t i = 0; i < n; ++i) {
      bool c = p.as<uint8_t>()[scalar_pred ? 0 : i] != 0;
      std::memcpy(t.data.data() + i * es, (c ? a : b).data.data() + i * es, es);
    }
    return t;
  }

  // reduction.zig:839-878 / 1157-1177: one output at a time, init first, then a left-to-right fold
  // over the reduced coordinates in row-major order of the reduced axes.
  Tensor reduce(const Op& op, const Tensor& x, const Tensor& init) {
    Tensor t = make(op.result);
    const auto& in_dims = x.type.dims;
    auto in_strides = row_major_strides(in_dims);
    std::vector<size_t> red, keep;
    for (size_t d = 0; d < in_dims.size(); ++d) {
      bool r = false;
      for (int64_t a : op.ints) r |= (a == (int64_t)d);
      (r ? red : keep).push_back(d);
    }
    uint64_t nout = t.n();
    uint64_t nred = 1;
    for (size_t d : red) nred *= (uint64_t)in_dims[d].extent;
    Reducer rk = (Reducer)op.code;
    DType dt = x.type.dtype;
    // Reduced offsets in fold order.
    std::vector<int64_t> roff(nred);
    for (uint64_t r = 0; r < nred; ++r) {
      uint64_t rem = r;
      int64_t off = 0;
      for (int k = (int)red.size() - 1; k >= 0; --k) {
        int64_t e = in_dims[red[k]].extent;
        off += (int64_t)(rem % e) * in_strides[red[k]];
        rem /= e;
      }
      roff[r] = off;
    }
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < (int64_t)nout; ++o) {
      uint64_t rem = o;
      int64_t base = 0;
      for (int k = (int)keep.size() - 1; k >= 0; --k) {
        int64_t e = in_dims[keep[k]].extent;
        base += (int64_t)(rem % e) * in_strides[keep[k]];
        rem /= e;
      }
      if (is_f32_domain(dt)) {
        float acc = (float)load_f(init, 0);
        if (dt == DType::f32) {
          const float* px = x.as<float>() + base;
          for (uint64_t r = 0; r < nred; ++r) {
            float val = px[roff[r]];
            acc = rk == Reducer::sum ? acc + val : rk == Reducer::max ? ref_max(acc, val) : ref_min(acc, val);
          }
        } else {
          for (uint64_t r = 0; r < nred; ++r) {
            float val = (float)load_f(x, base + roff[r]);
            acc = rk == Reducer::sum ? acc + val : rk == Reducer::max ? ref_max(acc, val) : ref_min(acc, val);
          }
        }
        store_f(t, o, acc);
      } else if (dt == DType::f64) {
        double acc = load_f(init, 0);
        for (uint64_t r = 0; r < nred; ++r) {
          double val = load_f(x, base + roff[r]);
          acc = rk == Reducer::sum ? acc + val : rk == Reducer::max ? ref_max(acc, val) : ref_min(acc, val);
        }
        store_f(t, o, acc);
      } else {
        bool uns = dtype_is_unsigned(dt);
        int64_t acc = load_i(init, 0);
        Binary b = rk == Reducer::sum ? Binary::add : rk == Reducer::max ? Binary::max : Binary::min;
        for (uint64_t r = 0; r < nred; ++r) acc = binary_int(b, acc, load_i(x, base + roff[r]), uns);
        store_i(t, o, acc);
      }
    }
    return t;
  }

  // dot.zig:2049-2115: per output a serial fold acc = acc + a*b over the contracted coordinates
  // (row-major in the listed contract-axis order), f32 accumulator for 16-bit inputs. The loop nest
  // keeps each output's k order while sweeping outputs of one lhs row together.
  Tensor dot(const Op& op, const Tensor& A, const Tensor& B) {
    Tensor t = make(op.result);
    const auto& ld = A.type.dims;
    const auto& rd = B.type.dims;
    auto ls = row_major_strides(ld), rs = row_major_strides(rd);
    std::vector<size_t> lfree, rfree;
    auto in = [](const std::vector<int64_t>& v, size_t d) {
      for (int64_t x : v)
        if (x == (int64_t)d) return true;
      return false;
    };
    for (size_t d = 0; d < ld.size(); ++d)
      if (!in(op.lhs_contract, d) && !in(op.lhs_batch, d)) lfree.push_back(d);
    for (size_t d = 0; d < rd.size(); ++d)
      if (!in(op.rhs_contract, d) && !in(op.rhs_batch, d)) rfree.push_back(d);
    auto enumerate = [](const std::vector<Dim>& dims, const std::vector<int64_t>& strides,
                        const std::vector<size_t>& axes) {
      uint64_t n = 1;
      for (size_t a : axes) n *= (uint64_t)dims[a].extent;
      std::vector<int64_t> off(n);
      for (uint64_t i = 0; i < n; ++i) {
        uint64_t rem = i;
        int64_t o = 0;
        for (int k = (int)axes.size() - 1; k >= 0; --k) {
          int64_t e = dims[axes[k]].extent;
          o += (int64_t)(rem % e) * strides[axes[k]];
          rem /= e;
        }
        off[i] = o;
      }
      return off;
    };
    std::vector<size_t> lb(op.lhs_batch.begin(), op.lhs_batch.end()), rb(op.rhs_batch.begin(), op.rhs_batch.end());
    std::vector<size_t> lc(op.lhs_contract.begin(), op.lhs_contract.end()),
        rc(op.rhs_contract.begin(), op.rhs_contract.end());
    auto lbo = enumerate(ld, ls, lb), rbo = enumerate(rd, rs, rb);
    auto lfo = enumerate(ld, ls, lfree), rfo = enumerate(rd, rs, rfree);
    auto lco = enumerate(ld, ls, lc), rco = enumerate(rd, rs, rc);
    uint64_t NB = lbo.size(), M = lfo.size(), N = rfo.size(), K = lco.size();
    DType dt = A.type.dtype;
    if (NB * M * N == 0) return t;
    if (is_f32_domain(dt)) {
      // Widen both operands to f32 once (exact), then fold.
      std::vector<float> a32(A.n()), b32(B.n());
      for (uint64_t i = 0; i < A.n(); ++i) a32[i] = (float)load_f(A, i);
      for (uint64_t i = 0; i < B.n(); ++i) b32[i] = (float)load_f(B, i);
#pragma omp parallel for collapse(2) schedule(static)
      for (int64_t b = 0; b < (int64_t)NB; ++b)
        for (int64_t m = 0; m < (int64_t)M; ++m) {
          std::vector<float> acc(N, 0.0f);
          int64_t abase = lbo[b] + lfo[m];
          for (uint64_t k = 0; k < K; ++k) {
            float av = a32[abase + lco[k]];
            const float* bp = b32.data() + rbo[b] + rco[k];
            for (uint64_t n = 0; n < N; ++n) {
              float prod = av * bp[rfo[n]];
              acc[n] = acc[n] + prod;
            }
          }
          uint64_t obase = ((uint64_t)b * M + m) * N;
          for (uint64_t n = 0; n < N; ++n) store_f(t, obase + n, acc[n]);
        }
    } else if (dt == DType::f64) {
      for (uint64_t b = 0; b < NB; ++b)
        for (uint64_t m = 0; m < M; ++m)
          for (uint64_t n = 0; n < N; ++n) {
            double acc = 0;
            for (uint64_t k = 0; k < K; ++k) {
              double prod = load_f(A, lbo[b] + lfo[m] + lco[k]) * load_f(B, rbo[b] + rfo[n] + rco[k]);
              acc = acc + prod;
            }
            store_f(t, (b * M + m) * N + n, acc);
          }
    } else {
      bool uns = dtype_is_unsigned(dt);
      for (uint64_t b = 0; b < NB; ++b)
        for (uint64_t m = 0; m < M; ++m)
          for (uint64_t n = 0; n < N; ++n) {
            int64_t acc = 0;
            for (uint64_t k = 0; k < K; ++k)
              acc = binary_int(Binary::add, acc,
                               binary_int(Binary::mul, load_i(A, lbo[b] + lfo[m] + lco[k]),
                                          load_i(B, rbo[b] + rfo[n] + rco[k]), uns),
                               uns);
            store_i(t, (b * M + m) * N + n, acc);
          }
    }
    return t;
  }

  // result[pre, j..., post] = input[pre, clamp(indices[j...]), post].
  Tensor gather(const Op& op, const Tensor& x, const Tensor& idx) {
    Tensor t = make(op.result);
    size_t axis = (size_t)op.axis;
    const auto& xd = x.type.dims;
    uint64_t pre = 1, post = 1;
    for (size_t d = 0; d < axis; ++d) pre *= (uint64_t)xd[d].extent;
    for (size_t d = axis + 1; d < xd.size(); ++d) post *= (uint64_t)xd[d].extent;
    int64_t ext = xd[axis].extent;
    uint64_t ni = idx.n();
    size_t es = dtype_size(x.type.dtype);
    for (uint64_t p = 0; p < pre; ++p)
      for (uint64_t j = 0; j < ni; ++j) {
        int64_t k = idx.as<int32_t>()[j];
        k = k < 0 ? 0 : (k > ext - 1 ? ext - 1 : k);
        std::memcpy(t.data.data() + ((p * ni + j) * post) * es, x.data.data() + ((p * ext + k) * post) * es,
                    post * es);
      }
    return t;
  }

  // result = input; result[pre, clamp(indices[j]), post] += updates[pre, j, post], updates in order.
  Tensor scatter_add(const Op& op, const Tensor& x, const Tensor& idx, const Tensor& upd) {
    Tensor t = x;
    size_t axis = (size_t)op.axis;
    const auto& xd = x.type.dims;
    uint64_t pre = 1, post = 1;
    for (size_t d = 0; d < axis; ++d) pre *= (uint64_t)xd[d].extent;
    for (size_t d = axis + 1; d < xd.size(); ++d) post *= (uint64_t)xd[d].extent;
    int64_t ext = xd[axis].extent;
    uint64_t ni = idx.n();
    bool fl = dtype_is_float(x.type.dtype), uns = dtype_is_unsigned(x.type.dtype);
    for (uint64_t p = 0; p < pre; ++p)
      for (uint64_t j = 0; j < ni; ++j) {
        int64_t k = idx.as<int32_t>()[j];
        k = k < 0 ? 0 : (k > ext - 1 ? ext - 1 : k);
        for (uint64_t q = 0; q < post; ++q) {
          uint64_t di = (p * ext + k) * post + q, si = (p * ni + j) * post + q;
          if (fl) {
            if (x.type.dtype == DType::f64) store_f(t, di, load_f(t, di) + load_f(upd, si));
            else store_f(t, di, (float)load_f(t, di) + (float)load_f(upd, si));
          } else {
            store_i(t, di, binary_int(Binary::add, load_i(t, di), load_i(upd, si), uns));
          }
        }
      }
    return t;
  }
};

int status_for(const Error& e) {
  switch (e.code) {
    case Err::UnsupportedVersion: return 2;
    case Err::Unsupported: return 7;
    default: return 1;
  }
}

}  // namespace

extern "C" {

// Same arguments and status numbers as accy_hip_run (src/tensor/session/session.zig:33-43).
int accy_cpu_run(const uint8_t* wire_bytes, size_t wire_len, const void* const* inputs, const size_t* input_lens,
                 size_t n_inputs, void* const* outputs, const size_t* output_lens, size_t n_outputs) {
  Program prog;
  try {
    prog = wire::decode(wire_bytes, wire_len);
  } catch (const Error& e) {
    g_error = e.what();
    return e.code == Err::UnsupportedVersion ? 2 : 1;
  }
  try {
    if (n_inputs != prog.params.size() || n_outputs != prog.outputs.size()) {
      g_error = "buffer count mismatch";
      return 4;
    }
    std::vector<Tensor> ins;
    for (size_t i = 0; i < n_inputs; ++i) {
      const Type& t = prog.type(prog.params[i]);
      if (input_lens[i] != t.bytes()) {
        g_error = "input " + std::to_string(i) + " size mismatch";
        return 4;
      }
      Tensor x;
      x.type = t;
      x.data.assign((const uint8_t*)inputs[i], (const uint8_t*)inputs[i] + input_lens[i]);
      ins.push_back(std::move(x));
    }
    for (size_t i = 0; i < n_outputs; ++i)
      if (output_lens[i] != prog.type(prog.outputs[i]).bytes()) {
        g_error = "output " + std::to_string(i) + " size mismatch";
        return 4;
      }
    auto outs = Evaluator(prog).run(std::move(ins));
    for (size_t i = 0; i < n_outputs; ++i) std::memcpy(outputs[i], outs[i].data.data(), output_lens[i]);
    return 0;
  } catch (const Error& e) {
    g_error = e.what();
    return status_for(e);
  } catch (const std::bad_alloc&) {
    g_error = "out of memory";
    return 6;
  } catch (const std::exception& e) {
    g_error = e.what();
    return 8;
  }
}

const char* accy_cpu_last_error(void) { return g_error.c_str(); }

void accy_cpu_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

int accy_cpu_max_threads(void) { return omp_get_max_threads(); }

// Scalar libm bindings, exposed so tests can compare the f32 transcendentals against closed forms.
float accy_cpu_unary_f32(int code, float x) { return unary_f32((Unary)code, x); }

// Decodes wire bytes with the shared codec and encodes the result again (tests check that the C++
// codec and the Python tracer's encoder agree byte for byte). Returns a status like accy_cpu_run.
int accy_cpu_wire_roundtrip(const uint8_t* wire_bytes, size_t wire_len, uint8_t* out, size_t cap, size_t* needed) {
  try {
    Program prog = wire::decode(wire_bytes, wire_len);
    std::vector<uint8_t> bytes = wire::encode(prog);
    if (needed) *needed = bytes.size();
    if (out && cap >= bytes.size()) std::memcpy(out, bytes.data(), bytes.size());
    return 0;
  } catch (const Error& e) {
    g_error = e.what();
    return e.code == Err::UnsupportedVersion ? 2 : 1;
  }
}

// Decodes wire bytes with the shared codec and writes the type the decoder's checked builder derived
// for every value, one line each ("<depth> <kind> <dtype>{name=extent,...}"), scan bodies after their
// scan at depth + 1. Tests compare these with the types the Python tracer derived on its own while
// recording, so a wrong derivation in the decoder (shared with the product) cannot go unseen.
static void dump_types(const Graph& g, int depth, std::string& out) {
  for (const Op& op : g.ops) {
    out += std::to_string(depth) + " " + kind_name(op.kind) + " " + op.result.str() + "\n";
    if (op.body) dump_types(*op.body, depth + 1, out);
  }
}

int accy_cpu_wire_types(const uint8_t* wire_bytes, size_t wire_len, char* out, size_t cap, size_t* needed) {
  try {
    Program prog = wire::decode(wire_bytes, wire_len);
    std::string text;
    dump_types(prog, 0, text);
    if (needed) *needed = text.size() + 1;
    if (out && cap > text.size()) std::memcpy(out, text.c_str(), text.size() + 1);
    return 0;
  } catch (const Error& e) {
    g_error = e.what();
    return e.code == Err::UnsupportedVersion ? 2 : 1;
  }
}

// Name of the error the last failing decode raised (e.g. "BadMagic").
const char* accy_cpu_error_name(void) {
  size_t colon = g_error.find(':');
  static thread_local std::string name;
  name = colon == std::string::npos ? g_error : g_error.substr(0, colon);
  return name.c_str();
}
}
