// Program -> kernel plan for gfx950.
//
// Fusion follows the reference's planning classes (src/preparation/fusion/pass.zig:234-292):
//  * elementwise and shape operations (unary, binary, compare, select, broadcast, broadcast_in_dim,
//    reshape, transpose, iota, splat constants, gather) are never materialised on their own; each
//    consumer evaluates them at its own index, as the reference's reduction prologues and dot
//    epilogues do (lowering/reduction.zig:881-901, lowering/elementwise.zig);
//  * reductions over trailing axes that share one row space fuse into a single row kernel, one
//    workgroup per row: several reductions in dependency order (max, then a sum that uses the max),
//    then the values of row shape and of full-row shape that depend on them — the row pipelines of
//    lowering/row.zig (logsumexp, softmax, RMS norm), here with no f32-only / cols%1024 limits;
//  * other reductions run as serial folds, one output per thread, in runCpu's exact order
//    (reduction.zig:1157-1190);
//  * contractions (dot_general, and sum-of-product reductions that are contractions) go to the MFMA
//    GEMM template, attention chains (dot -> scale -> [mask] -> softmax -> dot) to the fused attention
//    template; shapes those templates do not take fall back to a serial dot kernel with runCpu's
//    per-output k order (dot.zig:2049-2115).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <set>
#include <sstream>

#include "plan.hpp"
#include "lower_internal.hpp"

namespace accy {
namespace detail {

// ---------------------------------------------------------------------------------------------
// C types and literals
// ---------------------------------------------------------------------------------------------

const char* compute_type(DType d) {
  switch (d) {
    case DType::f16: case DType::bf16: case DType::f32: return "float";
    case DType::f64: return "double";
    case DType::i1: return "bool";
    case DType::i8: return "i8_t";
    case DType::i16: return "i16_t";
    case DType::i32: return "i32_t";
    case DType::i64: return "i64_t";
    case DType::u8: return "u8_t";
    case DType::u16: return "u16_t";
    case DType::u32: return "u32_t";
    case DType::u64: case DType::key: return "u64_t";
  }
  return "?";
}

const char* storage_type(DType d) {
  switch (d) {
    case DType::f16: case DType::bf16: return "u16_t";
    case DType::i1: return "u8_t";
    default: return compute_type(d);
  }
}

const char* unsigned_type(DType d) {
  switch (d) {
    case DType::i8: case DType::u8: return "u8_t";
    case DType::i16: case DType::u16: return "u16_t";
    case DType::i32: case DType::u32: return "u32_t";
    default: return "u64_t";
  }
}

bool is_float_domain(DType d) { return d == DType::f16 || d == DType::bf16 || d == DType::f32; }
bool is_int(DType d) { return dtype_is_signed(d) || dtype_is_unsigned(d) || d == DType::key; }

std::string round_to(DType d, const std::string& x) {
  if (d == DType::f16) return "accy::round_f16(" + x + ")";
  if (d == DType::bf16) return "accy::round_bf16(" + x + ")";
  return x;
}

static std::string hexf(double v, bool single) {
  if (std::isnan(v)) return single ? "__builtin_nanf(\"\")" : "__builtin_nan(\"\")";
  if (std::isinf(v)) return v > 0 ? (single ? "__builtin_inff()" : "__builtin_inf()")
                                   : (single ? "(-__builtin_inff())" : "(-__builtin_inf())");
  std::ostringstream os;
  os << std::hexfloat << v;
  std::string s = os.str();
  return single ? s + "f" : s;
}

// A constant element (raw storage bytes) written as a compute-domain literal.
std::string literal(DType d, const uint8_t* p) {
  switch (d) {
    case DType::f16: return hexf(f16_bits_to_f32((uint16_t)(p[0] | (p[1] << 8))), true);
    case DType::bf16: return hexf(bf16_bits_to_f32((uint16_t)(p[0] | (p[1] << 8))), true);
    case DType::f32: {
      float f;
      std::memcpy(&f, p, 4);
      return hexf(f, true);
    }
    case DType::f64: {
      double f;
      std::memcpy(&f, p, 8);
      return hexf(f, false);
    }
    case DType::i1: return p[0] ? "true" : "false";
    default: {
      uint64_t u = 0;
      size_t n = dtype_size(d);
      for (size_t i = 0; i < n; ++i) u |= (uint64_t)p[i] << (8 * i);
      if (dtype_is_signed(d) && n < 8 && (u >> (8 * n - 1)) & 1) u |= ~0ull << (8 * n);
      std::ostringstream os;
      os << "((" << compute_type(d) << ")" << u << "ull)";
      return os.str();
    }
  }
}

// ---------------------------------------------------------------------------------------------
// index expressions
// ---------------------------------------------------------------------------------------------

std::string offset_expr(const std::vector<std::string>& coords, const std::vector<int64_t>& strides) {
  std::string s;
  for (size_t d = 0; d < coords.size(); ++d) {
    if (strides[d] == 0 || coords[d] == "0") continue;
    std::string term = strides[d] == 1 ? coords[d] : coords[d] + "*" + std::to_string(strides[d]);
    s += s.empty() ? term : " + " + term;
  }
  return s.empty() ? "0" : "(" + s + ")";
}

std::vector<std::string> delinearize(const std::string& lin, const std::vector<Dim>& dims) {
  std::vector<std::string> c(dims.size());
  auto strides = row_major_strides(dims);
  for (size_t d = 0; d < dims.size(); ++d) {
    int64_t e = dims[d].extent;
    if (e == 1) {
      c[d] = "0";
      continue;
    }
    std::string q = strides[d] == 1 ? lin : "(" + lin + ")/" + std::to_string(strides[d]);
    c[d] = d == 0 ? (dims.size() == 1 ? lin : "(" + q + ")") : "((" + q + ")%" + std::to_string(e) + ")";
  }
  return c;
}

// ---------------------------------------------------------------------------------------------
// KernelWriter: builds one generated kernel
// ---------------------------------------------------------------------------------------------

KernelWriter::KernelWriter(const Graph& g, Slots& slots, const std::string& index_type)
    : itype(index_type), g_(g), slots_(slots) {}

std::string KernelWriter::arg(int slot, bool write) {
  for (size_t i = 0; i < args.size(); ++i)
    if (args[i] == slot) {
      if (write) writes[i] = true;
      return "a" + std::to_string(i);
    }
  args.push_back(slot);
  writes.push_back(write);
  return "a" + std::to_string(args.size() - 1);
}

std::string KernelWriter::tmp() { return "v" + std::to_string(ntmp_++); }

std::string KernelWriter::params() const {
  std::string s;
  for (size_t i = 0; i < args.size(); ++i) {
    const SlotInfo& si = slots_.plan.slots[(size_t)args[i]];
    if (i) s += ", ";
    s += writes[i] ? "" : "const ";
    s += storage_type(si.dtype);
    s += "* __restrict__ a" + std::to_string(i);
  }
  return s;
}

std::string KernelWriter::align_hints() const {
  std::string s;
  for (size_t i = 0; i < args.size(); ++i) {
    const SlotInfo& si = slots_.plan.slots[(size_t)args[i]];
    std::string t = std::string(writes[i] ? "" : "const ") + storage_type(si.dtype) + "*";
    s += "  a" + std::to_string(i) + " = (" + t + ")__builtin_assume_aligned(a" + std::to_string(i) + ", 16);\n";
  }
  return s;
}

std::string KernelWriter::load(int slot, const std::string& off, DType d) {
  std::string a = arg(slot, false);
  switch (d) {
    case DType::f16: return "accy::ld_f16(" + a + ", " + off + ")";
    case DType::bf16: return "accy::ld_bf16(" + a + ", " + off + ")";
    case DType::i1: return "accy::ld_i1(" + a + ", " + off + ")";
    default: return a + "[" + off + "]";
  }
}

std::string KernelWriter::load_at(int slot, const std::string& base, const std::string& idx, DType d) {
  std::string p = "(" + arg(slot, false) + " + " + base + ")";
  switch (d) {
    case DType::f16: return "accy::ld_f16(" + p + ", " + idx + ")";
    case DType::bf16: return "accy::ld_bf16(" + p + ", " + idx + ")";
    case DType::i1: return "accy::ld_i1(" + p + ", " + idx + ")";
    default: return p + "[" + idx + "]";
  }
}

std::string KernelWriter::quad_load(int slot, const std::string& var, const std::string& base, DType d, bool stream) {
  const std::string q = std::string("accy::Quad<") + storage_type(d) + ">";
  if (stream) return "const " + q + " " + var + " = accy::ld_quad_stream(" + arg(slot, false) + " + " + base + ");";
  return "const " + q + " " + var + " = *(const " + q + "*)(" + arg(slot, false) + " + " + base + ");";
}

std::string KernelWriter::quad_elem(const std::string& var, const std::string& idx, DType d) {
  const std::string e = var + ".v[" + idx + "]";
  switch (d) {
    case DType::f16: return "accy::f16_to_f32(" + e + ")";
    case DType::bf16: return "accy::bf16_to_f32(" + e + ")";
    case DType::i1: return "(" + e + " != 0)";
    default: return e;
  }
}

std::string KernelWriter::store(int slot, const std::string& off, DType d, const std::string& v) {
  std::string a = arg(slot, true);
  switch (d) {
    case DType::f16: return "accy::st_f16(" + a + ", " + off + ", " + v + ");";
    case DType::bf16: return "accy::st_bf16(" + a + ", " + off + ", " + v + ");";
    case DType::i1: return "accy::st_i1(" + a + ", " + off + ", " + v + ");";
    default: return a + "[" + off + "] = " + v + ";";
  }
}

std::string KernelWriter::value(uint32_t vid, const std::vector<std::string>& coords, Scope& sc) {
  std::string key = std::to_string(vid) + "@";
  for (const auto& c : coords) key += c + ",";
  auto it = sc.memo.find(key);
  if (it != sc.memo.end()) return it->second;
  std::string out;
  if (provide && provide(vid, coords, out)) {
    sc.memo[key] = out;
    return out;
  }
  const Op& op = g_.ops[vid];
  const Type& rt = op.result;
  DType d = rt.dtype;
  auto emit = [&](const std::string& expr) {
    std::string t = tmp();
    sc.out << sc.indent << "const " << compute_type(d) << " " << t << " = " << expr << ";\n";
    sc.memo[key] = t;
    return t;
  };
  int slot = slots_.available(vid);
  if (slot >= 0) {
    std::string off = offset_expr(coords, row_major_strides(rt.dims));
    std::string cached;
    if (leaf_hook && leaf_hook(slot, off, d, sc, cached)) {
      sc.memo[key] = cached;
      return cached;
    }
    return emit(load(slot, off, d));
  }
  switch (op.kind) {
    case Kind::constant: {
      if (is_splat_constant(op) || rt.elements() == 1)
        return emit(literal(d, (const uint8_t*)op.bytes.data()));
      int cs = slots_.constant(vid);
      return emit(load(cs, offset_expr(coords, row_major_strides(rt.dims)), d));
    }
    case Kind::iota: {
      std::string c = coords[(size_t)op.axis];
      return emit(round_to(d, "(" + std::string(compute_type(d)) + ")(" + c + ")"));
    }
    case Kind::unary: {
      std::string x = value(op.args[0], coords, sc);
      Unary u = (Unary)op.code;
      std::string e;
      if (is_float_domain(d) || d == DType::f64) {
        bool f = d != DType::f64;
        switch (u) {
          case Unary::neg: e = "-" + x; break;
          case Unary::abs: e = (f ? "fabsf(" : "fabs(") + x + ")"; break;
          case Unary::exp: e = (f ? "accy::exp_f32(" : "exp(") + x + ")"; break;
          case Unary::log: e = (f ? "logf(" : "log(") + x + ")"; break;
          case Unary::sqrt: e = (f ? "sqrtf(" : "sqrt(") + x + ")"; break;
          case Unary::tanh: e = (f ? "accy::tanh_f32(" : "tanh(") + x + ")"; break;
          case Unary::sin: e = (f ? "accy::sin_f32(" : "sin(") + x + ")"; break;
          case Unary::cos: e = (f ? "accy::cos_f32(" : "cos(") + x + ")"; break;
          case Unary::tan: e = (f ? "tanf(" : "tan(") + x + ")"; break;
        }
        return emit(round_to(d, e));
      }
      if (is_int(d)) {
        std::string T = compute_type(d), U = unsigned_type(d);
        if (u == Unary::neg) return emit("accy::wsub<" + T + "," + U + ">((" + T + ")0, " + x + ")");
        if (u == Unary::abs) {
          if (dtype_is_unsigned(d)) return emit(x);
          return emit("(" + x + " < 0 ? accy::wsub<" + T + "," + U + ">((" + T + ")0, " + x + ") : " + x + ")");
        }
      }
      fail(Err::Unsupported, std::string("unary op on ") + dtype_name(d));
    }
    case Kind::binary: {
      std::string x = value(op.args[0], coords, sc);
      std::string y = value(op.args[1], coords, sc);
      Binary b = (Binary)op.code;
      std::string e;
      if (is_float_domain(d) || d == DType::f64) {
        bool f = d != DType::f64;
        switch (b) {
          case Binary::add: e = x + " + " + y; break;
          case Binary::sub: e = x + " - " + y; break;
          case Binary::mul: e = x + " * " + y; break;
          case Binary::div: e = x + " / " + y; break;
          case Binary::max: e = (f ? "fmaxf(" : "fmax(") + x + ", " + y + ")"; break;
          case Binary::min: e = (f ? "fminf(" : "fmin(") + x + ", " + y + ")"; break;
          case Binary::pow: e = (f ? "powf(" : "pow(") + x + ", " + y + ")"; break;
        }
        return emit(round_to(d, e));
      }
      if (is_int(d)) {
        std::string T = compute_type(d), U = unsigned_type(d), tu = "<" + T + "," + U + ">";
        switch (b) {
          case Binary::add: return emit("accy::wadd" + tu + "(" + x + ", " + y + ")");
          case Binary::sub: return emit("accy::wsub" + tu + "(" + x + ", " + y + ")");
          case Binary::mul: return emit("accy::wmul" + tu + "(" + x + ", " + y + ")");
          case Binary::div: return emit("accy::idiv(" + x + ", " + y + ")");
          case Binary::max: return emit("accy::imax(" + x + ", " + y + ")");
          case Binary::min: return emit("accy::imin(" + x + ", " + y + ")");
          case Binary::pow: break;
        }
      }
      if (d == DType::i1) {
        switch (b) {
          case Binary::max: case Binary::add: return emit("(" + x + " || " + y + ")");
          case Binary::min: case Binary::mul: return emit("(" + x + " && " + y + ")");
          case Binary::sub: return emit("(" + x + " != " + y + ")");
          default: break;
        }
      }
      fail(Err::Unsupported, std::string("binary op on ") + dtype_name(d));
    }
    case Kind::compare: {
      std::string x = value(op.args[0], coords, sc);
      std::string y = value(op.args[1], coords, sc);
      static const char* ops[] = {"<", "<=", ">", ">=", "==", "!="};
      std::string t = tmp();
      sc.out << sc.indent << "const bool " << t << " = " << x << " " << ops[op.code] << " " << y << ";\n";
      sc.memo[key] = t;
      return t;
    }
    case Kind::select: {
      const Type& pt = g_.type(op.args[0]);
      std::vector<std::string> pc = pt.rank() == 0 ? std::vector<std::string>{} : coords;
      std::string p = value(op.args[0], pc, sc);
      std::string x = value(op.args[1], coords, sc);
      std::string y = value(op.args[2], coords, sc);
      return emit("(" + p + " ? " + x + " : " + y + ")");
    }
    case Kind::broadcast_in_dim: {
      const Type& it = g_.type(op.args[0]);
      std::vector<std::string> ic(it.rank());
      for (size_t j = 0; j < it.rank(); ++j) ic[j] = it.dims[j].extent == 1 ? "0" : coords[(size_t)op.ints[j]];
      std::string r = value(op.args[0], ic, sc);
      sc.memo[key] = r;
      return r;
    }
    case Kind::broadcast: {
      const Type& it = g_.type(op.args[0]);
      std::vector<std::string> ic;
      if (it.elements() == 1) {
        ic.assign(it.rank(), "0");
      } else if (it.elements() == rt.elements()) {
        ic = delinearize(offset_expr(coords, row_major_strides(rt.dims)), it.dims);
      } else {
        fail(Err::Unsupported, "broadcast of a non-splat operand");
      }
      std::string r = value(op.args[0], ic, sc);
      sc.memo[key] = r;
      return r;
    }
    case Kind::transpose: {
      const Type& it = g_.type(op.args[0]);
      std::vector<std::string> ic(it.rank());
      for (size_t k = 0; k < rt.rank(); ++k) ic[(size_t)op.ints[k]] = coords[k];
      std::string r = value(op.args[0], ic, sc);
      sc.memo[key] = r;
      return r;
    }
    case Kind::reshape: {
      const Type& it = g_.type(op.args[0]);
      std::vector<std::string> ic;
      bool same = it.rank() == rt.rank();
      for (size_t k = 0; same && k < rt.rank(); ++k) same = it.dims[k].extent == rt.dims[k].extent;
      if (same) ic = coords;
      else ic = delinearize(offset_expr(coords, row_major_strides(rt.dims)), it.dims);
      std::string r = value(op.args[0], ic, sc);
      sc.memo[key] = r;
      return r;
    }
    case Kind::gather: {
      // result[pre, j..., post] = input[pre, clamp(indices[j...]), post]
      const Type& it = g_.type(op.args[0]);
      const Type& xt = g_.type(op.args[1]);
      size_t axis = (size_t)op.axis, ri = xt.rank();
      std::vector<std::string> jc(coords.begin() + axis, coords.begin() + axis + ri);
      std::string idx = value(op.args[1], jc, sc);
      std::string cl = tmp();
      int64_t ext = it.dims[axis].extent;
      sc.out << sc.indent << "const " << itype << " " << cl << " = (" << itype << ")(" << idx << " < 0 ? 0 : ("
             << idx << " > " << (ext - 1) << " ? " << (ext - 1) << " : " << idx << "));\n";
      std::vector<std::string> ic(coords.begin(), coords.begin() + axis);
      ic.push_back(cl);
      ic.insert(ic.end(), coords.begin() + axis + ri, coords.end());
      std::string r = value(op.args[0], ic, sc);
      sc.memo[key] = r;
      return r;
    }
    default: break;
  }
  throw NotFusable(std::string("value %") + std::to_string(vid) + " (" + kind_name(op.kind) +
                   ") is not available in this kernel");
}

// ---------------------------------------------------------------------------------------------
// Slots
// ---------------------------------------------------------------------------------------------

Slots::Slots(const Graph& g, Plan& p) : plan(p), slot_of(g.ops.size(), -1), produced(g.ops.size(), false), g_(g) {}

int Slots::add(SlotInfo::Role role, int io, DType d, uint64_t bytes) {
  SlotInfo s;
  s.role = role;
  s.io_index = io;
  s.dtype = d;
  s.bytes = bytes;
  plan.slots.push_back(s);
  return (int)plan.slots.size() - 1;
}

int Slots::available(uint32_t vid) const { return produced[vid] ? slot_of[vid] : -1; }

int Slots::constant(uint32_t vid) {
  auto it = const_slot_.find(vid);
  if (it != const_slot_.end()) return it->second;
  const Op& op = g_.ops[vid];
  int s = add(SlotInfo::Const, -1, op.result.dtype, op.result.bytes());
  plan.slots[(size_t)s].data = op.bytes;
  const_slot_[vid] = s;
  return s;
}

}  // namespace detail
}  // namespace accy
