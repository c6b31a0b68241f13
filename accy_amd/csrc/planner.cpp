// Kernel formation: walks the program in operation order and turns every value that must live in a
// device buffer into a generated kernel. See lower.cpp for the fusion rules and the references.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <optional>
#include <functional>
#include <set>
#include <sstream>

#include "lower_internal.hpp"
#include "plan.hpp"
#include "tuning.hpp"

namespace accy {
using namespace detail;

namespace {

bool is_inlinable(Kind k) {
  switch (k) {
    case Kind::unary: case Kind::binary: case Kind::compare: case Kind::select: case Kind::broadcast:
    case Kind::broadcast_in_dim: case Kind::reshape: case Kind::transpose: case Kind::iota:
    case Kind::constant: case Kind::gather:
      return true;
    default:
      return false;
  }
}

// An offset of the form `(rest + c)` (c the innermost coordinate, stride 1; no other term mentions
// c), as `(rest) + c0`: where the VEC adjacent elements c0 .. c0 + VEC - 1 of one thread start.
std::optional<std::string> quad_base(const std::string& off) {
  if (off.size() < 2 || off.front() != '(' || off.back() != ')') return std::nullopt;
  std::string body = off.substr(1, off.size() - 2), rest;
  bool found = false;
  size_t pos = 0;
  while (pos <= body.size()) {
    size_t nx = body.find(" + ", pos);
    std::string term = body.substr(pos, nx == std::string::npos ? std::string::npos : nx - pos);
    bool has_c = false;
    for (size_t i = 0; i < term.size(); ++i) {
      bool ident_start = i == 0 || !(isalnum((unsigned char)term[i - 1]) || term[i - 1] == '_');
      bool ident_end = i + 1 == term.size() || !(isalnum((unsigned char)term[i + 1]) || term[i + 1] == '_');
      if (term[i] == 'c' && ident_start && ident_end) has_c = true;
    }
    if (term == "c" && !found) found = true;
    else if (has_c) return std::nullopt;
    else rest += (rest.empty() ? "" : " + ") + term;
    if (nx == std::string::npos) break;
    pos = nx + 3;
  }
  if (!found) return std::nullopt;
  return "(" + (rest.empty() ? std::string("0") : rest) + ") + c0";
}

uint64_t prod(const std::vector<Dim>& dims, size_t b, size_t e) {
  uint64_t n = 1;
  for (size_t i = b; i < e; ++i) n *= (uint64_t)dims[i].extent;
  return n;
}

// 32-bit indices while every element index plus one grid stride (at most 2^20 workgroups x 256
// threads = 2^28) stays below 2^31, so that no grid-stride loop's increment overflows.
std::string index_type(uint64_t max_elems) { return max_elems < (1ull << 31) - (1ull << 28) ? "i32_t" : "i64_t"; }

uint32_t grid_for(uint64_t work_items, uint32_t block, uint64_t cap = 1u << 20) {
  uint64_t g = (work_items + block - 1) / block;
  if (g == 0) g = 1;
  return (uint32_t)std::min<uint64_t>(g, cap);
}

// The body of a 64 x 64 tile of a transposing copy through LDS, for a kernel that has defined
// `const long r0, c0` (the tile's first r and c). The source's r axis is contiguous (element (r, c)
// at src[r + c * sc]), the destination's c axis (element (r, c) at dst[r * ds + c]); extents R and
// C. Tiles are read along r and written along c, so both sides touch whole lines. `et` is the
// element's storage type. With `epl` > 1 (4, 8 or 16; R, C, sc and ds multiples of it and both bases
// aligned to it), each lane moves `epl` consecutive elements per access, 16 bytes for 1- to 4-byte
// elements; otherwise one element per access. `epl` comes from transpose_lanes, which gives 8 only
// for 2-byte elements; the 8 path packs two elements per 32-bit LDS word and assumes that size.
std::string transpose_tile(const std::string& et, int64_t R, int64_t C, int64_t sc, int64_t ds, const std::string& src,
                           const std::string& dst, int epl) {
  std::ostringstream k;
  const std::string r = std::to_string(R) + "L", c = std::to_string(C) + "L";
  if (epl == 8) {
    // 2-byte elements: an LDS word holds the elements of columns 2p and 2p + 1 at one r (the lower
    // column in the low half, as in memory), so each LDS access moves two elements. A lane loads 8
    // r of two adjacent columns and writes 8 words; on the way out it reads 4 words of one r (8
    // consecutive c) for one 16-byte store. Pitch 33 words.
    k << "  __shared__ u32_t tile[64][33];\n"
      << "  typedef " << et << " V __attribute__((ext_vector_type(8)));\n"
      << "  typedef u32_t W __attribute__((ext_vector_type(4)));\n"
      << "  const int t = (threadIdx.x & 7) * 8, p = threadIdx.x >> 3;\n"
      << "  if (r0 + t < " << r << " && c0 + 2 * p < " << c << ") {\n"
      << "    const V a = *(const V*)&" << src << "[r0 + t + (c0 + 2 * p) * " << sc << "L];\n"
      << "    const V b = *(const V*)&" << src << "[r0 + t + (c0 + 2 * p + 1) * " << sc << "L];\n"
      << "#pragma unroll\n    for (int j = 0; j < 8; ++j) tile[t + j][p] = (u32_t)(u16_t)a[j] | ((u32_t)(u16_t)b[j] << 16);\n"
      << "  }\n"
      << "  __syncthreads();\n"
      << "  const int w = (threadIdx.x & 7) * 4;\n"
      << "  for (int r = threadIdx.x >> 3; r < 64; r += 32)\n"
      << "    if (r0 + r < " << r << " && c0 + 2 * w < " << c << ") {\n"
      << "      const W v = {tile[r][w], tile[r][w + 1], tile[r][w + 2], tile[r][w + 3]};\n"
      << "      *(W*)&" << dst << "[(r0 + r) * " << ds << "L + c0 + 2 * w] = v;\n"
      << "    }\n";
    return k.str();
  }
  k << "  __shared__ " << et << " tile[64][65];\n";
  if (epl > 1) {
    const int lanes = 64 / epl, step = 256 / lanes;  // lanes per 64 elements of r; columns per pass
    k << "  typedef " << et << " V __attribute__((ext_vector_type(" << epl << ")));\n"
      << "  const int t = (threadIdx.x % " << lanes << ") * " << epl << ", q = threadIdx.x / " << lanes << ";\n"
      << "  for (int c = q; c < 64; c += " << step << ")\n"
      << "    if (r0 + t < " << r << " && c0 + c < " << c << ") {\n"
      << "      const V v = *(const V*)&" << src << "[r0 + t + (c0 + c) * " << sc << "L];\n"
      << "#pragma unroll\n      for (int j = 0; j < " << epl << "; ++j) tile[c][t + j] = v[j];\n"
      << "    }\n"
      << "  __syncthreads();\n"
      << "  for (int r = q; r < 64; r += " << step << ")\n"
      << "    if (r0 + r < " << r << " && c0 + t < " << c << ") {\n"
      << "      V v;\n"
      << "#pragma unroll\n      for (int j = 0; j < " << epl << "; ++j) v[j] = tile[t + j][r];\n"
      << "      *(V*)&" << dst << "[(r0 + r) * " << ds << "L + c0 + t] = v;\n"
      << "    }\n";
  } else {
    k << "  const int t = threadIdx.x & 63, q = threadIdx.x >> 6;\n"
      << "  for (int c = q; c < 64; c += 4)\n"
      << "    if (r0 + t < " << r << " && c0 + c < " << c << ") tile[c][t] = " << src << "[r0 + t + (c0 + c) * " << sc
      << "L];\n"
      << "  __syncthreads();\n"
      << "  for (int r = q; r < 64; r += 4)\n"
      << "    if (r0 + r < " << r << " && c0 + t < " << c << ") " << dst << "[(r0 + r) * " << ds << "L + c0 + t] = tile[t][r];\n";
  }
  return k.str();
}

// Elements per lane access of a tiled transpose: 16 bytes' worth for elements of at most 4 bytes
// (4 for 8-byte elements), when every extent, stride and offset in `multiples` is a multiple of it;
// then 4; else 1.
int transpose_lanes(size_t elem_bytes, const std::vector<int64_t>& multiples) {
  for (int e : {std::max<int>(4, (int)(16 / elem_bytes)), 4}) {
    bool ok = true;
    for (int64_t x : multiples) ok = ok && x % e == 0;
    if (ok) return e;
  }
  return 1;
}

const char* reducer_op(Reducer r) {
  switch (r) {
    case Reducer::sum: return "accy::SumOp()";
    case Reducer::max: return "accy::MaxOp()";
    case Reducer::min: return "accy::MinOp()";
  }
  return "";
}

// Accumulator type of a reduction: f32 for 16-bit floats (reduction.zig:847, 861 widen f16), the
// unsigned twin for integer sums so wrap-around is defined.
std::string acc_type(DType d, Reducer r) {
  if (is_int(d) && r == Reducer::sum) return unsigned_type(d);
  return compute_type(d);
}

// The step of a serial fold (fold and chunked fold kernels): as fold_step, with float max / min that
// keep the later element on ties, as runCpu's fold does (accy::fold_max / fold_min).
std::string serial_fold_step(DType d, Reducer r, const std::string& acc, const std::string& x);

std::string fold_step(DType d, Reducer r, const std::string& acc, const std::string& x) {
  if (is_float_domain(d)) {
    if (r == Reducer::sum) return acc + " + " + x;
    return std::string(r == Reducer::max ? "fmaxf(" : "fminf(") + acc + ", " + x + ")";
  }
  if (d == DType::f64) {
    if (r == Reducer::sum) return acc + " + " + x;
    return std::string(r == Reducer::max ? "fmax(" : "fmin(") + acc + ", " + x + ")";
  }
  if (r == Reducer::sum) return acc + " + (" + acc_type(d, r) + ")" + x;
  return std::string(r == Reducer::max ? "accy::imax(" : "accy::imin(") + acc + ", " + x + ")";
}

std::string serial_fold_step(DType d, Reducer r, const std::string& acc, const std::string& x) {
  if ((is_float_domain(d) || d == DType::f64) && r != Reducer::sum)
    return std::string(r == Reducer::max ? "accy::fold_max(" : "accy::fold_min(") + acc + ", " + x + ")";
  return fold_step(d, r, acc, x);
}

class Planner {
 public:
  Planner(const Graph& g, const LowerOptions& o) : g_(g), opt_(o), slots_(g, plan_) {
    for (const Op& op : g.ops) max_elems_ = std::max<uint64_t>(max_elems_, op.result.elements());
  }

  Plan run() {
    size_t n = g_.ops.size();
    live_.assign(n, false);
    needed_.assign(n, false);
    done_.assign(n, false);
    mark_live();
    for (size_t i = 0; i < g_.params.size(); ++i) {
      uint32_t p = g_.params[i];
      const Type& t = g_.type(p);
      int s = slots_.add(SlotInfo::Input, (int)i, t.dtype, t.bytes());
      slots_.slot_of[p] = s;
      slots_.produced[p] = true;
      done_[p] = true;
      plan_.input_slots.push_back(s);
    }
    // Output slots: the first occurrence of a computed value is written in place; parameters and
    // repeated outputs are copied at the end.
    std::vector<std::pair<int, int>> copies;  // (source value, output position)
    plan_.output_slots.assign(g_.outputs.size(), -1);
    for (size_t i = 0; i < g_.outputs.size(); ++i) {
      uint32_t v = g_.outputs[i];
      const Type& t = g_.type(v);
      int s = slots_.add(SlotInfo::Output, (int)i, t.dtype, t.bytes());
      plan_.output_slots[i] = s;
      if (g_.ops[v].kind == Kind::parameter || slots_.slot_of[v] >= 0) {
        copies.push_back({(int)v, (int)i});
      } else {
        slots_.slot_of[v] = s;
        needed_[v] = true;
      }
    }
    match_attentions();
    mark_gemm_operands();
    for (uint32_t v = 0; v < n; ++v) {
      if (!live_[v] || done_[v]) continue;
      process(v);
    }
    for (auto& c : copies) {
      uint32_t v = (uint32_t)c.first;
      int src = slots_.available(v);
      if (src < 0 && g_.ops[v].kind == Kind::constant) {
        map_into(v, plan_.output_slots[(size_t)c.second]);
        continue;
      }
      if (src < 0) fail(Err::Unsupported, "output source not computed");
      Step st;
      st.type = Step::Copy;
      st.copy.src = src;
      st.copy.dst = plan_.output_slots[(size_t)c.second];
      st.copy.bytes = g_.type(v).bytes();
      if (st.copy.bytes) plan_.steps.push_back(st);
    }
    return std::move(plan_);
  }

 private:
  const Graph& g_;
  LowerOptions opt_;
  Plan plan_;
  Slots slots_;
  std::vector<bool> live_, needed_, done_;
  int counter_ = 0;
  uint64_t max_elems_ = 1;

  // Index arithmetic is 32-bit unless some value of the program has 2^31 or more elements.
  std::string itype() const { return index_type(max_elems_); }

  void process(uint32_t v) {
    const Op& op = g_.ops[v];
    switch (op.kind) {
      case Kind::parameter: break;
      case Kind::reduce:
        if (!mulsum(v) && !row_group(v)) fold(v);
        break;
      case Kind::dot_general: dot(v); break;
      case Kind::scatter_add: scatter_add(v); break;
      case Kind::scan: scan(v); break;
      case Kind::projection: break;  // written by its scan's loop step
      case Kind::custom_call: case Kind::sparse_cross_entropy:  // sparse_cross_entropy is expanded before planning
        fail(Err::Unsupported, std::string(kind_name(op.kind)) + " is not supported by the HIP target");
      default:
        if (needed_[v]) map(v);
        break;
    }
  }

  void mark_live() {
    std::vector<uint32_t> stack(g_.outputs.begin(), g_.outputs.end());
    while (!stack.empty()) {
      uint32_t v = stack.back();
      stack.pop_back();
      if (live_[v]) continue;
      live_[v] = true;
      for (uint32_t a : g_.ops[v].args) stack.push_back(a);
    }
  }

  int temp_slot(uint32_t v) {
    if (slots_.slot_of[v] < 0) {
      const Type& t = g_.type(v);
      slots_.slot_of[v] = slots_.add(SlotInfo::Temp, -1, t.dtype, t.bytes());
    }
    return slots_.slot_of[v];
  }

  std::string name(const char* klass, uint32_t v) {
    return std::string("accy_") + klass + "_" + std::to_string(counter_++) + "_v" + std::to_string(v);
  }

  void push(KernelStep k, const KernelWriter& w) {
    k.args = w.args;
    double bytes = 0;
    for (size_t i = 0; i < w.args.size(); ++i) bytes += (double)plan_.slots[(size_t)w.args[i]].bytes;
    k.algorithmic_bytes = bytes;
    Step st;
    st.type = Step::Kernel;
    st.kernel = std::move(k);
    plan_.steps.push_back(std::move(st));
  }

  void finish(uint32_t v) {
    done_[v] = true;
    slots_.produced[v] = true;
  }

  // Slot of value a, materialised by a map kernel when so far it is only evaluated inline.
  int materialize(uint32_t a) {
    int s = slots_.available(a);
    if (s >= 0) return s;
    if (!is_inlinable(g_.ops[a].kind)) fail(Err::Unsupported, "value not computed before its use");
    map(a);
    return slots_.available(a);
  }

  // ---- scan: the body's own plan, run as a host loop over two sets of carry buffers ----
  // The scan's value is carry 0 and projection i is carry i (builder.zig:899-990); a carry without a
  // reader gets no result slot.
  void scan(uint32_t v) {
    const Op& op = g_.ops[v];
    Step st;
    st.type = Step::Loop;
    LoopStep& L = st.loop;
    L.body = op.body;
    LowerOptions bo = opt_;
    bo.force_candidate.clear();
    L.plan = std::make_shared<const Plan>(lower(*op.body, bo));
    L.length = op.axis;
    for (uint32_t a : op.args) L.init_slots.push_back(materialize(a));
    L.result_slots.assign(op.args.size(), -1);
    std::vector<CopyStep> extra;  // a second projection of a carry that is also a program output
    auto take = [&](uint32_t value, size_t carry) {
      if (L.result_slots[carry] >= 0 && slots_.slot_of[value] < 0) {
        slots_.slot_of[value] = L.result_slots[carry];  // another projection of the same carry: same slot
        finish(value);
        return;
      }
      const int s = slots_.slot_of[value] >= 0 ? slots_.slot_of[value] : temp_slot(value);
      if (L.result_slots[carry] < 0) {
        L.result_slots[carry] = s;
      } else {
        CopyStep c;
        c.src = L.result_slots[carry];
        c.dst = s;
        c.bytes = g_.type(value).bytes();
        extra.push_back(c);
      }
      finish(value);
    };
    take(v, 0);
    for (uint32_t u = v + 1; u < (uint32_t)g_.ops.size(); ++u) {
      const Op& p = g_.ops[u];
      if (p.kind == Kind::projection && p.args[0] == v && live_[u]) take(u, (size_t)p.index);
    }
    plan_.steps.push_back(std::move(st));
    for (const CopyStep& c : extra) {
      if (!c.bytes) continue;
      Step cs;
      cs.type = Step::Copy;
      cs.copy = c;
      plan_.steps.push_back(cs);
    }
  }

  // ---- map: out[i] = value at i ----
  void map(uint32_t v) {
    map_into(v, slots_.slot_of[v] >= 0 ? slots_.slot_of[v] : temp_slot(v));
    finish(v);
  }

  void map_into(uint32_t v, int slot) {
    const Type& t = g_.type(v);
    uint64_t nel = t.elements();
    if (nel == 0) return;
    View pv;
    if (resolve_view(v, pv) && permute_copy(v, slot, pv)) return;
    KernelWriter w(g_, slots_, itype());
    std::ostringstream body;
    const uint32_t B = 256;
    const int64_t inner = t.rank() ? t.dims.back().extent : 1;
    std::string nm = name("map", v);
    std::ostringstream src;
    // The kernel's parameters are known once its body is written.
    auto head = [&]() {
      return "extern \"C\" __global__ void __launch_bounds__(" + std::to_string(B) + ") " + nm + "(" + w.params() +
             ") {\n  typedef " + w.itype + " I;\n";
    };
    KernelStep k;
    if (t.rank() >= 1 && inner % 4 == 0) {
      // Four consecutive elements per thread (the innermost extent is a multiple of 4, so they share
      // their outer coordinates): c0 is the innermost coordinate of the first, c = c0 + u. A leaf read
      // at `rest + c` is loaded once for the four as one vector load at the top of the iteration,
      // non-temporal when this kernel reads each of its elements once (as many elements as the
      // output, so no axis is broadcast); the four stores are adjacent.
      std::vector<Dim> outer(t.dims.begin(), t.dims.end() - 1);
      std::vector<std::string> coords =
          outer.empty() ? std::vector<std::string>{} : delinearize("(i0 / " + std::to_string(inner) + ")", outer);
      coords.push_back("c");
      std::string hoisted;
      std::map<std::string, std::string> hoisted_var;
      int nq = 0;
      w.leaf_hook = [&](int s, const std::string& off, DType d, Scope& sc, std::string& out) -> bool {
        std::optional<std::string> base = quad_base(off);
        if (!base) return false;
        const std::string key = std::to_string(s) + "|" + off;
        auto hv = hoisted_var.find(key);
        if (hv == hoisted_var.end()) {
          const bool stream = plan_.slots[(size_t)s].bytes / dtype_size(d) == nel;
          const std::string q = "q" + std::to_string(nq++);
          hoisted += "    " + w.quad_load(s, q, *base, d, stream) + "\n";
          hv = hoisted_var.emplace(key, q).first;
        }
        const std::string tmp = w.tmp();
        sc.out << sc.indent << "const " << compute_type(d) << " " << tmp << " = " << KernelWriter::quad_elem(hv->second, "u", d)
               << ";\n";
        out = tmp;
        return true;
      };
      Scope sc(body, "      ");
      std::string x = w.value(v, coords, sc);
      body << sc.indent << w.store(slot, "i0 + u", t.dtype, x) << "\n";
      src << head() << w.align_hints() << "  for (I i0 = ((I)blockIdx.x * " << B << " + (I)threadIdx.x) * 4; i0 < (I)" << nel
          << "; i0 += (I)gridDim.x * " << 4 * B << ") {\n"
          << "    const I c0 = " << (outer.empty() ? std::string("i0") : "(i0) % " + std::to_string(inner)) << ";\n"
          << hoisted << "#pragma unroll\n    for (int u = 0; u < 4; ++u) {\n      const I c = c0 + u;\n"
          << body.str() << "    }\n  }\n}\n";
      // One vector of four per thread where the grid allows (a streaming copy of 1 GiB measured 6.3
      // TB/s moved this way against 5.6 with four iterations per thread).
      k.grid[0] = grid_for(nel / 4, B);
    } else {
      Scope sc(body, "    ");
      std::vector<std::string> coords = delinearize("i", t.dims);
      std::string x = w.value(v, coords, sc);
      body << sc.indent << w.store(slot, "i", t.dtype, x) << "\n";
      src << head() << "  for (I i = (I)blockIdx.x * " << B << " + threadIdx.x; i < (I)" << nel << "; i += (I)gridDim.x * " << B
          << ") {\n"
          << body.str() << "  }\n}\n";
      k.grid[0] = grid_for(nel, B, 65536);
    }
    k.source = src.str();
    k.name = nm;
    k.block[0] = B;
    k.klass = "map";
    k.label = "map:%" + std::to_string(v);
    push(std::move(k), w);
  }

  // ---- fold: one output per thread, serial left-to-right over the reduced index ----
  void fold(uint32_t v) {
    const Op& op = g_.ops[v];
    const Type& in = g_.type(op.args[0]);
    const Type& rt = op.result;
    int out = slots_.slot_of[v] >= 0 ? slots_.slot_of[v] : temp_slot(v);
    uint64_t nout = rt.elements();
    if (nout == 0) {
      finish(v);
      return;
    }
    std::vector<size_t> red, keep;
    for (size_t d = 0; d < in.rank(); ++d)
      (std::find(op.ints.begin(), op.ints.end(), (int64_t)d) != op.ints.end() ? red : keep).push_back(d);
    std::vector<Dim> rdims, kdims;
    for (size_t d : red) rdims.push_back(in.dims[d]);
    for (size_t d : keep) kdims.push_back(in.dims[d]);
    uint64_t nred = prod(rdims, 0, rdims.size());
    Reducer r = (Reducer)op.code;
    DType d = rt.dtype;
    // Few outputs over a long reduced range: one serial fold per output cannot fill the GPU (and keeps
    // too few loads in flight), so the range is folded in chunks and the chunks' partials folded in
    // order (fold_chunked).
    if (nred >= 1024 && nout * nred >= (1ull << 22) && nout < (1ull << 18) && chunk_identity(d, r)) {
      fold_chunked(v, out, in, red, keep, rdims, kdims, nout, nred, r, d);
      finish(v);
      return;
    }
    KernelWriter w(g_, slots_, itype());
    std::ostringstream body;
    Scope outer(body, "    ");
    std::vector<std::string> kc = delinearize("o", kdims);
    std::string init = w.value(op.args[1], {}, outer);
    std::string at = acc_type(d, r);
    body << "    " << at << " acc = (" << at << ")" << init << ";\n";
    body << "    for (I r = 0; r < (I)" << nred << "; ++r) {\n";
    Scope inner(body, "      ");
    std::vector<std::string> rc = delinearize("r", rdims);
    std::vector<std::string> full(in.rank());
    for (size_t i = 0; i < red.size(); ++i) full[red[i]] = rc[i];
    for (size_t i = 0; i < keep.size(); ++i) full[keep[i]] = kc[i];
    std::string x = w.value(op.args[0], full, inner);
    body << "      acc = " << serial_fold_step(d, r, "acc", x) << ";\n    }\n";
    std::string res = is_int(d) ? "(" + std::string(compute_type(d)) + ")acc" : round_to(d, "acc");
    body << "    " << w.store(out, "o", d, res) << "\n";
    const uint32_t B = 256;
    std::string nm = name("fold", v);
    std::ostringstream src;
    src << "extern \"C\" __global__ void __launch_bounds__(" << B << ") " << nm << "(" << w.params() << ") {\n"
        << "  typedef " << w.itype << " I;\n"
        << "  for (I o = (I)blockIdx.x * " << B << " + threadIdx.x; o < (I)" << nout << "; o += (I)gridDim.x * "
        << B << ") {\n"
        << body.str() << "  }\n}\n";
    KernelStep k;
    k.source = src.str();
    k.name = nm;
    k.grid[0] = grid_for(nout, B, 65536);
    k.block[0] = B;
    k.klass = "fold";
    k.label = "fold:%" + std::to_string(v);
    push(std::move(k), w);
    finish(v);
  }

  // The value a chunk's fold starts from, so that folding the chunks' partials in order from the
  // program's init gives the serial fold's result: -0 for a float sum (x + -0 = x for every x,
  // including -0), NaN for a float max / min (fold_max / fold_min skip a NaN second operand and return
  // the second operand when the first is NaN, so NaN is the absent element; ties keep the later
  // element, which the in-order combination of the chunks preserves), 0 for a
  // wrapping integer sum, the type's extreme for an integer max / min. Integer folds and float max /
  // min are then bit-identical to the serial fold; a float sum is associated differently (within the
  // reductions' 1e-5 relative bound). Empty for other dtypes.
  static std::optional<std::string> chunk_identity(DType d, Reducer r) {
    if (is_float_domain(d)) return std::string(r == Reducer::sum ? "-0.0f" : "__builtin_nanf(\"\")");
    if (d == DType::f64) return std::string(r == Reducer::sum ? "-0.0" : "__builtin_nan(\"\")");
    if (r == Reducer::sum && (d == DType::i32 || d == DType::u32 || d == DType::i64 || d == DType::u64))
      return "(" + acc_type(d, r) + ")0";
    const bool mx = r == Reducer::max;
    switch (d) {
      case DType::i32: return std::string(mx ? "(-2147483647 - 1)" : "2147483647");
      case DType::u32: return std::string(mx ? "0u" : "4294967295u");
      case DType::i64: return std::string(mx ? "(-9223372036854775807LL - 1)" : "9223372036854775807LL");
      case DType::u64: return std::string(mx ? "0ull" : "18446744073709551615ull");
      default: return std::nullopt;
    }
  }

  // Partial dtype of a chunked fold: f32 for the 16-bit floats and f32, f64, the unsigned type for a
  // wrapping integer sum, the dtype itself for an integer max / min.
  static DType partial_dtype(DType d, Reducer r) {
    if (is_float_domain(d)) return DType::f32;
    if (r == Reducer::sum && d == DType::i32) return DType::u32;
    if (r == Reducer::sum && d == DType::i64) return DType::u64;
    return d;
  }

  // Kernel 1: output o, chunk s (blockIdx.y) folds reduced indices [s * chunk, (s + 1) * chunk) in
  // order from the chunk identity into part[s * nout + o]. Kernel 2: each output folds its S partials
  // in chunk order from the program's init, then rounds once (16-bit dtypes) and stores.
  void fold_chunked(uint32_t v, int out, const Type& in, const std::vector<size_t>& red, const std::vector<size_t>& keep,
                    const std::vector<Dim>& rdims, const std::vector<Dim>& kdims, uint64_t nout, uint64_t nred, Reducer r,
                    DType d) {
    const Op& op = g_.ops[v];
    const uint32_t B = 256;
    uint64_t S = std::max<uint64_t>(2, ((1ull << 20) + nout - 1) / nout);
    S = std::min<uint64_t>(S, std::min<uint64_t>(nred / 256, 65535));
    const uint64_t chunk = (nred + S - 1) / S;
    S = (nred + chunk - 1) / chunk;
    const DType pd = partial_dtype(d, r);
    const std::string at = acc_type(d, r);
    const int part = slots_.add(SlotInfo::Temp, -1, pd, S * nout * dtype_size(pd));
    {
      KernelWriter w(g_, slots_, itype());
      std::ostringstream body;
      std::vector<std::string> kc = delinearize("o", kdims), rc = delinearize("r", rdims);
      std::vector<std::string> full(in.rank());
      for (size_t i = 0; i < red.size(); ++i) full[red[i]] = rc[i];
      for (size_t i = 0; i < keep.size(); ++i) full[keep[i]] = kc[i];
      body << "    " << at << " acc = " << *chunk_identity(d, r) << ";\n"
           << "    const I r0 = s * (I)" << chunk << ";\n"
           << "    const I r1 = r0 + (I)" << chunk << " < (I)" << nred << " ? r0 + (I)" << chunk << " : (I)" << nred << ";\n"
           << "#pragma unroll 8\n    for (I r = r0; r < r1; ++r) {\n";
      Scope inner(body, "      ");
      std::string x = w.value(op.args[0], full, inner);
      body << "      acc = " << serial_fold_step(d, r, "acc", x) << ";\n    }\n"
           << "    " << w.store(part, "s * (I)" + std::to_string(nout) + " + o", pd, "acc") << "\n";
      std::string nm = name("fold_chunks", v);
      std::ostringstream src;
      src << "extern \"C\" __global__ void __launch_bounds__(" << B << ") " << nm << "(" << w.params() << ") {\n"
          << "  typedef " << w.itype << " I;\n  const I s = (I)blockIdx.y;\n"
          << "  for (I o = (I)blockIdx.x * " << B << " + threadIdx.x; o < (I)" << nout << "; o += (I)gridDim.x * " << B
          << ") {\n" << body.str() << "  }\n}\n";
      KernelStep k;
      k.source = src.str();
      k.name = nm;
      k.grid[0] = grid_for(nout, B, 65536);
      k.grid[1] = (uint32_t)S;
      k.block[0] = B;
      k.klass = "fold";
      k.label = "fold:%" + std::to_string(v) + " chunks";
      push(std::move(k), w);
    }
    {
      KernelWriter w(g_, slots_, itype());
      std::ostringstream body;
      Scope outer(body, "    ");
      std::string init = w.value(op.args[1], {}, outer);
      body << "    " << at << " acc = (" << at << ")" << init << ";\n"
           << "    for (I s = 0; s < (I)" << S << "; ++s) acc = "
           << serial_fold_step(d, r, "acc", w.load(part, "s * (I)" + std::to_string(nout) + " + o", pd)) << ";\n";
      std::string res = is_int(d) ? "(" + std::string(compute_type(d)) + ")acc" : round_to(d, "acc");
      body << "    " << w.store(out, "o", d, res) << "\n";
      std::string nm = name("fold", v);
      std::ostringstream src;
      src << "extern \"C\" __global__ void __launch_bounds__(" << B << ") " << nm << "(" << w.params() << ") {\n"
          << "  typedef " << w.itype << " I;\n"
          << "  for (I o = (I)blockIdx.x * " << B << " + threadIdx.x; o < (I)" << nout << "; o += (I)gridDim.x * " << B
          << ") {\n" << body.str() << "  }\n}\n";
      KernelStep k;
      k.source = src.str();
      k.name = nm;
      k.grid[0] = grid_for(nout, B, 65536);
      k.block[0] = B;
      k.klass = "fold";
      k.label = "fold:%" + std::to_string(v);
      push(std::move(k), w);
    }
  }

  // ---- row group: fused reductions over trailing axes of one row space, one workgroup per row ----
  struct RowShape {
    std::vector<Dim> K, T;
  };

  bool row_shape(uint32_t v, RowShape& rs) const {
    const Op& op = g_.ops[v];
    if (op.kind != Kind::reduce) return false;
    const Type& in = g_.type(op.args[0]);
    std::vector<int64_t> red = op.ints;
    std::sort(red.begin(), red.end());
    size_t rank = in.rank(), nr = red.size();
    if (nr == 0) return false;
    for (size_t i = 0; i < nr; ++i)
      if (red[i] != (int64_t)(rank - nr + i)) return false;
    rs.K.assign(in.dims.begin(), in.dims.begin() + (rank - nr));
    rs.T.assign(in.dims.begin() + (rank - nr), in.dims.end());
    DType d = op.result.dtype;
    return is_float_domain(d) || d == DType::f64 || is_int(d);
  }

  struct RowKernel {
    std::vector<uint32_t> reduces, row_vals, full_vals;
  };

  bool row_group(uint32_t r0) {
    if (!opt_.allow_row) return false;
    RowShape rs;
    if (!row_shape(r0, rs)) return false;
    uint64_t tn = prod(rs.T, 0, rs.T.size()), kn = prod(rs.K, 0, rs.K.size());
    if (tn < 64 || kn == 0) return false;
    RowKernel rk;
    rk.reduces.push_back(r0);
    if (!try_row(rs, rk)) return false;
    size_t n = g_.ops.size();
    for (uint32_t v = r0 + 1; v < n; ++v) {
      if (!live_[v] || done_[v]) continue;
      RowShape o;
      if (g_.ops[v].kind == Kind::reduce && row_shape(v, o) && o.K == rs.K && o.T == rs.T) {
        rk.reduces.push_back(v);
        if (!try_row(rs, rk)) rk.reduces.pop_back();
      }
    }
    std::vector<Dim> full = rs.K;
    full.insert(full.end(), rs.T.begin(), rs.T.end());
    for (uint32_t v = r0 + 1; v < n; ++v) {
      if (!live_[v] || done_[v] || !needed_[v] || !is_inlinable(g_.ops[v].kind)) continue;
      const auto& dims = g_.type(v).dims;
      if (dims == rs.K) {
        rk.row_vals.push_back(v);
        if (!try_row(rs, rk)) rk.row_vals.pop_back();
      } else if (dims == full) {
        rk.full_vals.push_back(v);
        if (!try_row(rs, rk)) rk.full_vals.pop_back();
      }
    }
    for (uint32_t v : rk.reduces) temp_slot(v);
    for (uint32_t v : rk.row_vals) temp_slot(v);
    for (uint32_t v : rk.full_vals) temp_slot(v);
    KernelStep k = gen_row(rs, rk, true);
    push_row(std::move(k));
    for (uint32_t v : rk.reduces) finish(v);
    for (uint32_t v : rk.row_vals) finish(v);
    for (uint32_t v : rk.full_vals) finish(v);
    return true;
  }

  std::vector<int> last_args_;

  void push_row(KernelStep k) {
    k.args = last_args_;
    double bytes = 0;
    for (int s : k.args) bytes += (double)plan_.slots[(size_t)s].bytes;
    k.algorithmic_bytes = bytes;
    Step st;
    st.type = Step::Kernel;
    st.kernel = std::move(k);
    plan_.steps.push_back(std::move(st));
  }

  bool try_row(const RowShape& rs, const RowKernel& rk) {
    try {
      gen_row(rs, rk, false);
      return true;
    } catch (const NotFusable&) {
      return false;
    }
  }

  KernelStep gen_row(const RowShape& rs, const RowKernel& rk, bool commit) {
    uint64_t tn = prod(rs.T, 0, rs.T.size()), kn = prod(rs.K, 0, rs.K.size());
    const uint32_t VEC = tn % 4 == 0 ? 4 : 1;
    uint64_t lanes = (tn + VEC - 1) / VEC;
    uint32_t B = lanes >= 256 ? 256 : (uint32_t)std::max<uint64_t>(64, (lanes + 63) / 64 * 64);
    uint64_t E = (tn + (uint64_t)B * VEC - 1) / ((uint64_t)B * VEC);
    size_t passes = rk.reduces.size() + (rk.full_vals.empty() ? 0 : 1);
    // A row read by several passes is kept in registers when each thread holds at most 64 of its
    // elements; a row too long for that with 256 threads takes 512 or 1024 threads if that makes it
    // fit (read once instead of once per pass; four waves per SIMD still have 128 registers each).
    if (passes >= 2 && E * VEC > 64) {
      for (uint32_t wide : {512u, 1024u}) {
        const uint64_t e = (tn + (uint64_t)wide * VEC - 1) / ((uint64_t)wide * VEC);
        if (e * VEC <= 64) {
          B = wide;
          E = e;
          break;
        }
      }
    }
    bool unrolled = E * VEC <= 64;
    bool cache = unrolled && passes >= 2;
    bool guard = tn % ((uint64_t)B * VEC) != 0;
    KernelWriter w(g_, slots_, itype());
    std::vector<std::string> kc = delinearize("row", rs.K);
    std::vector<std::string> tc = delinearize("c", rs.T);
    std::vector<std::string> full = kc;
    full.insert(full.end(), tc.begin(), tc.end());
    // Row-varying leaves loaded by more than one pass are kept in registers.
    std::map<std::string, std::set<int>> leaf_use;
    std::map<std::string, std::string> leaf_array;
    std::map<std::string, int> leaf_first;
    int cur_pass = 0;
    std::string decls;
    std::set<std::string> declared;
    if (commit) {
      KernelStep probe = gen_row(rs, rk, false);
      (void)probe;
      leaf_use = probe_use_;
      int na = 0;
      for (auto& [key, uses] : leaf_use) {
        if (cache && uses.size() >= 2) {
          leaf_array[key] = "cache" + std::to_string(na++);
          leaf_first[key] = *uses.begin();
        }
      }
    }
    std::map<std::string, std::set<int>> use_record;
    // A load whose offset is `rest + c` (c the row's element index, rank-1 row) is written as
    // (ptr + rest + c0)[u] so that the VEC adjacent loads of one thread merge into one vector load.
    // The `rest` of an offset `(rest + c)` (empty optional when the offset has another form).
    auto row_rest = [&](const std::string& off) -> std::optional<std::string> {
      if (VEC == 1 || tc.size() != 1 || tc[0] != "c") return std::nullopt;
      return quad_base(off);
    };
    auto direct_load = [&](int slot, const std::string& off, DType d) -> std::string {
      const std::optional<std::string> base = row_rest(off);
      return base ? w.load_at(slot, *base, "u", d) : w.load(slot, off, d);
    };
    // Without a tail guard, a leaf read at `rest + c` is loaded for the thread's VEC elements at once,
    // at the top of the element iteration (one aligned vector load per input, issued before any of
    // the iteration's arithmetic), and each element takes its lane.
    const bool hoist = VEC == 4 && !guard;
    std::string hoisted;
    std::map<std::string, std::string> hoisted_var;
    int nquad = 0;
    // A leaf is streamed (loaded with the non-temporal hint) when this kernel reads each of its
    // elements exactly once: its buffer holds as many elements as the kernel's rows x row length and
    // its offset depends on the row (a buffer reached through broadcast_in_dim covers a subset of the
    // loop's axes, so an equal element count means no axis is broadcast and no element is shared
    // between rows), and one pass reads it (or the row is cached in registers after the first).
    auto mentions_row = [](const std::string& off) {
      for (size_t p = off.find("row"); p != std::string::npos; p = off.find("row", p + 1)) {
        const bool start = p == 0 || !(isalnum((unsigned char)off[p - 1]) || off[p - 1] == '_');
        const bool end = p + 3 == off.size() || !(isalnum((unsigned char)off[p + 3]) || off[p + 3] == '_');
        if (start && end) return true;
      }
      return false;
    };
    auto streamed = [&](int slot, const std::string& off, DType d, const std::string& key) {
      if (!commit) return false;
      const auto use = leaf_use.find(key);
      const bool once = leaf_array.count(key) > 0 || (use != leaf_use.end() && use->second.size() == 1);
      const uint64_t elems = plan_.slots[(size_t)slot].bytes / dtype_size(d);
      return once && elems == kn * tn && mentions_row(off);
    };
    // The hoisted vector load of a leaf for this iteration (emitted once per pass), as the lane `u`.
    auto hoisted_elem = [&](int slot, const std::string& base, DType d, const std::string& key, bool stream) {
      auto hv = hoisted_var.find(key);
      if (hv == hoisted_var.end()) {
        std::string q = "q" + std::to_string(nquad++);
        hoisted += "      " + w.quad_load(slot, q, base, d, stream) + "\n";
        hv = hoisted_var.emplace(key, q).first;
      }
      return KernelWriter::quad_elem(hv->second, "u", d);
    };
    w.leaf_hook = [&](int slot, const std::string& off, DType d, Scope& sc, std::string& out) -> bool {
      bool varies = false;
      for (const auto& t : tc)
        if (t != "0" && off.find(t) != std::string::npos) varies = true;
      if (!varies) return false;
      std::string key = std::to_string(slot) + "|" + off;
      use_record[key].insert(cur_pass);
      auto it = leaf_array.find(key);
      if (it == leaf_array.end()) {
        std::string t = w.tmp();
        std::optional<std::string> base = hoist ? row_rest(off) : std::nullopt;
        std::string val = base ? hoisted_elem(slot, *base, d, key, streamed(slot, off, d, key)) : direct_load(slot, off, d);
        sc.out << sc.indent << "const " << compute_type(d) << " " << t << " = " << val << ";\n";
        out = t;
        return true;
      }
      std::string elem = it->second + "[e * " + std::to_string(VEC) + " + u]";
      if (leaf_first[key] == cur_pass) {
        // The cache is filled by the first pass; a streamed leaf through the hoisted vector load.
        std::optional<std::string> base = hoist && streamed(slot, off, d, key) ? row_rest(off) : std::nullopt;
        sc.out << sc.indent << elem << " = " << (base ? hoisted_elem(slot, *base, d, key, true) : direct_load(slot, off, d))
               << ";\n";
        if (declared.insert(key).second)
          decls += "    " + std::string(compute_type(d)) + " " + it->second + "[" + std::to_string(E * VEC) + "];\n";
      }
      out = elem;
      return true;
    };
    std::vector<std::string> red_var(rk.reduces.size());
    size_t avail = 0;
    w.provide = [&](uint32_t vid, const std::vector<std::string>& coords, std::string& out) -> bool {
      for (size_t j = 0; j < rk.reduces.size(); ++j) {
        if (rk.reduces[j] != vid) continue;
        if (j >= avail || coords != kc) throw NotFusable("reduction used outside its row");
        out = red_var[j];
        return true;
      }
      const Op& op = g_.ops[vid];
      if (!is_inlinable(op.kind) && slots_.available(vid) < 0) throw NotFusable("value not produced yet");
      return false;
    };
    std::ostringstream body;
    // Element loop: fully unrolled when the thread's elements are cached in registers across passes;
    // otherwise unrolled by a few iterations (all of them would keep every hoisted load live at once).
    // Launch candidates when not cached: the unroll factor (first = default); the source carries a
    // placeholder until the candidate is chosen.
    static const char* const kUnrollMark = "#pragma unroll ACCY_ELEMENT_UNROLL\n";
    const std::vector<int> unroll_candidates =
        cache ? std::vector<int>{0} : (unrolled ? std::vector<int>{4, 2, 1, 8} : std::vector<int>{2, 1, 4});
    std::string unroll = cache ? "#pragma unroll\n" : kUnrollMark;
    std::string loop_head_a, loop_head_b;
    {
      std::ostringstream la, lb;
      la << unroll << "    for (int e = 0; e < " << E << "; ++e) {\n"
         << "      const I c0 = ((I)e * " << B << " + (I)threadIdx.x) * " << VEC << ";\n";
      lb << "#pragma unroll\n"
         << "      for (int u = 0; u < " << VEC << "; ++u) {\n"
         << "        const I c = c0 + u;\n";
      if (guard) lb << "        if (c < (I)" << tn << ") {\n";
      loop_head_a = la.str();
      loop_head_b = lb.str();
    }
    // One element loop: head, the pass's hoisted loads, per-element code, tail.
    auto emit_loop = [&](const std::string& inner_code, const std::string& tail) {
      body << loop_head_a << hoisted << loop_head_b << inner_code << tail;
      hoisted.clear();
      hoisted_var.clear();
    };
    std::string loop_tail = guard ? "        }\n      }\n    }\n" : "      }\n    }\n";
    std::string lds_decl;
    for (size_t j = 0; j < rk.reduces.size(); ++j) {
      cur_pass = (int)j;
      const Op& op = g_.ops[rk.reduces[j]];
      Reducer r = (Reducer)op.code;
      DType d = op.result.dtype;
      std::string at = acc_type(d, r);
      Scope pre(body, "    ");
      std::string init = w.value(op.args[1], {}, pre);
      std::string acc = "acc" + std::to_string(j);
      body << "    " << at << " " << acc << " = (" << at << ")" << init << ";\n";
      std::ostringstream ib;
      Scope inner(ib, guard ? "          " : "        ");
      std::string x = w.value(op.args[0], full, inner);
      ib << inner.indent << acc << " = " << fold_step(d, r, acc, x) << ";\n";
      emit_loop(ib.str(), loop_tail);
      std::string lds = "lds" + std::to_string(j);
      lds_decl += "  __shared__ " + at + " " + lds + "[" + std::to_string(std::max<uint32_t>(B / 64, 1)) + "];\n";
      body << "    " << acc << " = accy::block_reduce<" << B << ">(" << acc << ", " << reducer_op(r) << ", " << lds
           << ");\n";
      red_var[j] = "red" + std::to_string(j);
      std::string res = is_int(d) ? "(" + std::string(compute_type(d)) + ")" + acc : round_to(d, acc);
      body << "    const " << compute_type(d) << " " << red_var[j] << " = " << res << ";\n";
      if (commit) body << "    if (threadIdx.x == 0) " << w.store(slots_.slot_of[rk.reduces[j]], "row", d, red_var[j]) << "\n";
      avail = j + 1;
    }
    if (!rk.row_vals.empty()) {
      body << "    if (threadIdx.x == 0) {\n";
      Scope sc(body, "      ");
      for (uint32_t v : rk.row_vals) {
        std::string x = w.value(v, kc, sc);
        if (commit) body << "      " << w.store(slots_.slot_of[v], "row", g_.type(v).dtype, x) << "\n";
      }
      body << "    }\n";
    }
    if (!rk.full_vals.empty()) {
      cur_pass = (int)rk.reduces.size();
      std::ostringstream ib;
      Scope sc(ib, guard ? "          " : "        ");
      for (uint32_t v : rk.full_vals) {
        std::string x = w.value(v, full, sc);
        if (commit) ib << sc.indent << w.store(slots_.slot_of[v], "row * (I)" + std::to_string(tn) + " + c", g_.type(v).dtype, x) << "\n";
      }
      emit_loop(ib.str(), loop_tail);
    }
    probe_use_ = use_record;
    KernelStep k;
    if (!commit) return k;
    std::string nm = name("row", rk.reduces[0]);
    std::ostringstream src;
    src << "extern \"C\" __global__ void __launch_bounds__(" << B << ") " << nm << "(" << w.params() << ") {\n"
        << "  typedef " << w.itype << " I;\n"
        << w.align_hints() << lds_decl << "  for (I row = blockIdx.x; row < (I)" << kn << "; row += gridDim.x) {\n"
        << decls << body.str() << "  }\n}\n";
    k.source = src.str();
    k.grid[0] = (uint32_t)std::min<uint64_t>(kn, 1u << 20);
    if (unroll_candidates.size() > 1) {
      k.tuning_key = tuning_key("row", k.source, "rows=" + std::to_string(kn) + ",cols=" + std::to_string(tn));
      k.candidate_count = (uint32_t)unroll_candidates.size();
      k.candidate = candidate_for(k.tuning_key, k.candidate_count);
      const std::string pragma = "#pragma unroll " + std::to_string(unroll_candidates[k.candidate]) + "\n";
      for (size_t at = k.source.find(kUnrollMark); at != std::string::npos; at = k.source.find(kUnrollMark, at))
        k.source.replace(at, std::strlen(kUnrollMark), pragma);
    }
    k.name = nm;
    k.block[0] = B;
    k.klass = "row";
    k.label = "row:%" + std::to_string(rk.reduces[0]);
    last_args_ = w.args;
    return k;
  }

  std::map<std::string, std::set<int>> probe_use_;

  // ---- launch tuning ----
  size_t kernel_index() const {
    size_t n = 0;
    for (const Step& st : plan_.steps) n += st.type == Step::Kernel ? 1 : 0;
    return n;
  }
  // Key of a tunable kernel: device family, class, fingerprint of its default source and a readable
  // shape.
  static std::string tuning_key(const std::string& klass, const std::string& source, const std::string& shape) {
    return "gfx950/" + klass + "/" + fingerprint(source) + "/" + shape;
  }
  // Candidate for the next kernel step: forced (measurement), else the table's selection, else 0.
  uint32_t candidate_for(const std::string& key, uint32_t count) const {
    if (count <= 1) return 0;
    auto f = opt_.force_candidate.find(kernel_index());
    if (f != opt_.force_candidate.end()) return f->second < count ? f->second : 0;
    if (opt_.tuning)
      if (auto sel = opt_.tuning->find(key, count)) return sel->candidate;
    return 0;
  }

  // ---- strided views: a value that is a transpose / rename / broadcast of a buffer ----
  struct View {
    int slot = -1;
    int64_t offset = 0;
    std::vector<int64_t> strides;  // per dim of the viewed value, in elements
  };

  bool resolve_view(uint32_t v, View& out) const {
    int s = slots_.available(v);
    const Op& op = g_.ops[v];
    const Type& t = op.result;
    if (s >= 0) {
      out.slot = s;
      out.offset = 0;
      out.strides = row_major_strides(t.dims);
      return true;
    }
    View in;
    switch (op.kind) {
      case Kind::transpose:
        if (!resolve_view(op.args[0], in)) return false;
        out = in;
        for (size_t k = 0; k < t.rank(); ++k) out.strides[k] = in.strides[(size_t)op.ints[k]];
        return true;
      case Kind::reshape: {
        const Type& it = g_.type(op.args[0]);
        if (it.rank() != t.rank()) return false;
        for (size_t k = 0; k < t.rank(); ++k)
          if (it.dims[k].extent != t.dims[k].extent) return false;
        return resolve_view(op.args[0], out);
      }
      case Kind::broadcast_in_dim: {
        if (!resolve_view(op.args[0], in)) return false;
        const Type& it = g_.type(op.args[0]);
        out.slot = in.slot;
        out.offset = in.offset;
        out.strides.assign(t.rank(), 0);
        for (size_t j = 0; j < op.ints.size(); ++j)
          if (it.dims[j].extent != 1) out.strides[(size_t)op.ints[j]] = in.strides[j];
        return true;
      }
      default:
        return false;
    }
  }

  // A value that is a permutation of a buffer (a transpose view) whose innermost axis is strided in
  // the source while another axis r is contiguous there: a copy through LDS, one 64 x 64 tile of
  // (r, innermost) per workgroup, read along r and written along the innermost axis, so both sides
  // touch whole lines (an element-wise map would read one line per element). The other axes are
  // enumerated by blockIdx.y. Raw storage is copied, so any dtype.
  bool permute_copy(uint32_t v, int slot, const View& pv) {
    const Type& t = g_.type(v);
    const size_t n = t.rank();
    if (n < 2) return false;
    const int64_t sc = pv.strides[n - 1];
    if (sc == 1 || sc == 0 || t.dims[n - 1].extent < 16) return false;
    size_t r = n;
    for (size_t a = 0; a + 1 < n; ++a)
      if (pv.strides[a] == 1 && t.dims[a].extent > 1) r = a;
    if (r == n) return false;
    const std::vector<int64_t> ds = row_major_strides(t.dims);
    int64_t outer = 1;
    for (size_t a = 0; a + 1 < n; ++a)
      if (a != r) outer *= t.dims[a].extent;
    if (outer > 65535) return false;
    const int64_t er = t.dims[r].extent, ec = t.dims[n - 1].extent, tc = (ec + 63) / 64;
    if (((er + 63) / 64) * tc >= (int64_t)1 << 24) return false;  // a launch holds fewer than 2^32 work items
    KernelWriter w(g_, slots_, "i64_t");
    const std::string src = w.arg(pv.slot, false), dst = w.arg(slot, true);
    const std::string T = storage_type(t.dtype);
    std::ostringstream k;
    const std::string nm = name("permute", v);
    k << "extern \"C\" __global__ void __launch_bounds__(256) " << nm << "(" << w.params() << ") {\n"
      << "  long o = blockIdx.y, so = " << pv.offset << "L, dof = 0;\n";
    for (size_t a = n - 1; a-- > 0;) {
      if (a == r) continue;
      k << "  { const long x = o % " << t.dims[a].extent << "L; o /= " << t.dims[a].extent << "L; so += x * "
        << pv.strides[a] << "L; dof += x * " << ds[a] << "L; }\n";
    }
    std::vector<int64_t> multiples = {er, ec, sc, pv.offset};
    for (size_t a = 0; a + 1 < n; ++a) {
      if (a != r) multiples.push_back(pv.strides[a]);
      multiples.push_back(ds[a]);
    }
    const int epl = transpose_lanes(dtype_size(t.dtype), multiples);
    k << "  const long r0 = (long)(blockIdx.x / " << tc << ") * 64, c0 = (long)(blockIdx.x % " << tc << ") * 64;\n"
      << transpose_tile(T, er, ec, sc, ds[r], "(" + src + " + so)", "(" + dst + " + dof)", epl) << "}\n";
    KernelStep ks;
    ks.source = k.str();
    ks.name = nm;
    ks.grid[0] = (uint32_t)(((er + 63) / 64) * tc);
    ks.grid[1] = (uint32_t)outer;
    ks.block[0] = 256;
    ks.klass = "map";
    ks.label = "permute:%" + std::to_string(v);
    ks.algorithmic_bytes = 2.0 * (double)t.bytes();
    push(std::move(ks), w);
    return true;
  }

  // Collapses a group of dims (in the given order) into one extent and stride, if the group is
  // contiguous in the view; an empty group is extent 1, stride 0.
  static bool flatten(const std::vector<Dim>& dims, const std::vector<int64_t>& strides,
                      const std::vector<size_t>& group, int64_t& extent, int64_t& stride) {
    extent = 1;
    stride = 0;
    bool first = true;
    for (size_t gi = group.size(); gi-- > 0;) {
      size_t d = group[gi];
      int64_t e = dims[d].extent;
      if (e == 1) continue;
      if (first) {
        stride = strides[d];
        first = false;
      } else if (strides[d] != stride * extent) {
        return false;
      }
      extent *= e;
    }
    return true;
  }

  // The axes of one operand group (batch, rows or contraction) in the order that flattens the
  // group's index, with their strides in the operand; neighbours that are contiguous are merged.
  struct Group {
    std::vector<int64_t> ext, str;  // runs, outermost first

    static Group make(const std::vector<Dim>& dims, const std::vector<int64_t>& strides, const std::vector<size_t>& idx) {
      Group g;
      for (size_t d : idx) {
        if (dims[d].extent == 1) continue;
        if (!g.ext.empty() && g.str.back() == strides[d] * dims[d].extent) {
          g.ext.back() *= dims[d].extent;
          g.str.back() = strides[d];
        } else {
          g.ext.push_back(dims[d].extent);
          g.str.push_back(strides[d]);
        }
      }
      return g;
    }
    int64_t extent() const {
      int64_t e = 1;
      for (int64_t x : ext) e *= x;
      return e;
    }
    bool single() const { return ext.size() <= 1; }
    int64_t stride() const { return ext.empty() ? 0 : str[0]; }
    // The innermost run: (extent, stride).
    int64_t inner_ext() const { return ext.empty() ? 1 : ext.back(); }
    int64_t inner_str() const { return ext.empty() ? 0 : str.back(); }
    bool strides_multiple_of(int64_t q) const {
      for (int64_t x : str)
        if (x % q != 0) return false;
      return true;
    }
    // Device function returning the element offset of flattened index i.
    std::string fn(const std::string& name) const {
      std::ostringstream s;
      s << "  static __device__ __forceinline__ long " << name << "(long i) { return 0L";
      int64_t inner = 1;
      for (size_t r = ext.size(); r-- > 0;) {
        s << " + ";
        std::string idx = inner == 1 ? "i" : "(i / " + std::to_string(inner) + "L)";
        if (r > 0) idx = "(" + idx + " % " + std::to_string(ext[r]) + "L)";
        s << idx << " * " << str[r] << "L";
        inner *= ext[r];
      }
      s << "; }\n";
      return s.str();
    }
  };

  struct GemmShape {
    int64_t batch = 1, m = 1, n = 1, k = 1;
    int64_t a_b = 0, a_m = 0, a_k = 0, b_b = 0, b_k = 0, b_n = 0;  // single strides (when !multi)
    Group ga_b, ga_m, ga_k, gb_b, gb_k, gb_n;
    bool multi = false;
    View a, b;
  };

  bool gemm_shape(const Op& op, GemmShape& gs) const {
    const Type& L = g_.type(op.args[0]);
    const Type& R = g_.type(op.args[1]);
    if (!resolve_view(op.args[0], gs.a) || !resolve_view(op.args[1], gs.b)) return false;
    auto in = [](const std::vector<int64_t>& a, size_t d) { return std::find(a.begin(), a.end(), (int64_t)d) != a.end(); };
    std::vector<size_t> lb(op.lhs_batch.begin(), op.lhs_batch.end()), rb(op.rhs_batch.begin(), op.rhs_batch.end());
    std::vector<size_t> lc(op.lhs_contract.begin(), op.lhs_contract.end()),
        rc(op.rhs_contract.begin(), op.rhs_contract.end());
    std::vector<size_t> lf, rf;
    for (size_t i = 0; i < L.rank(); ++i)
      if (!in(op.lhs_contract, i) && !in(op.lhs_batch, i)) lf.push_back(i);
    for (size_t i = 0; i < R.rank(); ++i)
      if (!in(op.rhs_contract, i) && !in(op.rhs_batch, i)) rf.push_back(i);
    // Batch and contraction axes pair up one to one.
    for (size_t i = 0; i < lc.size(); ++i)
      if (L.dims[lc[i]].extent != R.dims[rc[i]].extent) return false;
    for (size_t i = 0; i < lb.size(); ++i)
      if (L.dims[lb[i]].extent != R.dims[rb[i]].extent) return false;
    // Size-one axes drop out; a batch or contraction axis of extent > 1 on one side only cannot be.
    gs.ga_b = Group::make(L.dims, gs.a.strides, lb);
    gs.gb_b = Group::make(R.dims, gs.b.strides, rb);
    gs.ga_m = Group::make(L.dims, gs.a.strides, lf);
    gs.gb_n = Group::make(R.dims, gs.b.strides, rf);
    gs.ga_k = Group::make(L.dims, gs.a.strides, lc);
    gs.gb_k = Group::make(R.dims, gs.b.strides, rc);
    gs.batch = gs.ga_b.extent();
    gs.m = gs.ga_m.extent();
    gs.n = gs.gb_n.extent();
    gs.k = gs.ga_k.extent();
    if (gs.gb_b.extent() != gs.batch || gs.gb_k.extent() != gs.k) return false;
    // Pairwise merging can differ between the two sides; the offset functions decompose the same
    // flattened index either way, since merged runs are row-major over the same logical axes.
    gs.multi = !(gs.ga_b.single() && gs.gb_b.single() && gs.ga_m.single() && gs.gb_n.single() && gs.ga_k.single() &&
                 gs.gb_k.single());
    gs.a_b = gs.ga_b.stride();
    gs.b_b = gs.gb_b.stride();
    gs.a_m = gs.ga_m.stride();
    gs.b_n = gs.gb_n.stride();
    gs.a_k = gs.ga_k.stride();
    gs.b_k = gs.gb_k.stride();
    return true;
  }

  // Direct-to-LDS tile sizes for the 16-bit kernel (0: not applicable).
  static int dma_rows(int64_t extent) { return extent % 256 == 0 ? 256 : (extent % 128 == 0 ? 128 : 0); }

  // Operand layouts the direct-to-LDS kernel can stage: K-contiguous (the innermost contraction run
  // has stride 1 and whole 32-wide k tiles) or row-contiguous (the innermost row run has stride 1
  // and whole row tiles); every other stride and the offset 16-byte aligned.
  static bool dma_operand(const Group& rows, const Group& k, const Group& batch, int64_t offset, int tile, bool& kc) {
    if (!rows.strides_multiple_of(1) || offset % 8 != 0) return false;
    auto aligned8 = [](const Group& g, bool skip_inner) {
      for (size_t i = 0; i < g.str.size(); ++i) {
        if (skip_inner && i + 1 == g.str.size()) continue;
        if (g.str[i] % 8 != 0) return false;
      }
      return true;
    };
    if (!aligned8(batch, false)) return false;
    if (k.inner_str() == 1 && k.inner_ext() % 32 == 0 && aligned8(k, true) && aligned8(rows, false)) {
      kc = true;
      return true;
    }
    if (rows.inner_str() == 1 && rows.inner_ext() % tile == 0 && aligned8(rows, true) && aligned8(k, false)) {
      kc = false;
      return true;
    }
    return false;
  }

  bool dma_eligible(const GemmShape& gs, int& dm, int& dn, bool& a_kc, bool& b_kc) const {
    // whole K steps of 32, at least as many as pipeline stages
    if (gs.k % 32 != 0 || gs.k < 128 || std::getenv("ACCY_GEMM_NO_DMA")) return false;
    dm = dma_rows(gs.m);
    dn = dma_rows(gs.n);
    if (dm && dn)
      return dma_operand(gs.ga_m, gs.ga_k, gs.ga_b, gs.a.offset, dm, a_kc) &&
             dma_operand(gs.gb_n, gs.gb_k, gs.gb_b, gs.b.offset, dn, b_kc);
    // M or N not a multiple of 128: single-axis groups with extents a multiple of 8, tiles that reach
    // past the end (the kernel clamps those loads to the last row / chunk and stores only in range).
    if (gs.multi || gs.m % 8 != 0 || gs.n % 8 != 0) return false;
    dm = dm ? dm : (gs.m > 128 ? 256 : 128);
    dn = dn ? dn : (gs.n > 128 ? 256 : 128);
    return dma_operand(gs.ga_m, gs.ga_k, gs.ga_b, gs.a.offset, 8, a_kc) &&
           dma_operand(gs.gb_n, gs.gb_k, gs.gb_b, gs.b.offset, 8, b_kc);
  }

  // The f32 MFMA kernel's operand layouts: A K-contiguous, B N-contiguous, rows 16-byte aligned.
  static bool f32_layout_ok(const GemmShape& gs) {
    auto ok4 = [](int64_t x) { return x % 4 == 0; };
    return gs.a_k == 1 && gs.b_n == 1 && ok4(gs.a_m) && ok4(gs.b_k) && ok4(gs.a_b) && ok4(gs.b_b) &&
           ok4(gs.a.offset) && ok4(gs.b.offset);
  }

  // Copies an f32 operand view (batch x R x C with strides sb, sr, sc from offset `off` of `slot`) into
  // a new contiguous temporary [batch][R][C] and returns its slot. One workgroup per 64 x 64 tile: when
  // the rows are the contiguous axis (sr == 1, a transpose) the tile goes through LDS, read along r and
  // written along c, so both sides touch whole lines; otherwise element by element along c.
  int pack_f32(int slot, int64_t off, int64_t batch, int64_t R, int64_t C, int64_t sb, int64_t sr, int64_t sc) {
    const int dst = slots_.add(SlotInfo::Temp, -1, DType::f32, (uint64_t)(batch * R * C) * 4);
    KernelWriter w(g_, slots_, "i64_t");
    const std::string src = w.arg(slot, false), out = w.arg(dst, true);
    const std::string nm = name("pack", (uint32_t)dst);
    std::ostringstream k;
    const int64_t tr = (R + 63) / 64, tc = (C + 63) / 64;
    k << "extern \"C\" __global__ void __launch_bounds__(256) " << nm << "(" << w.params() << ") {\n"
      << "  const long b = blockIdx.y, r0 = (long)(blockIdx.x / " << tc << ") * 64, c0 = (long)(blockIdx.x % " << tc << ") * 64;\n"
      << "  const float* __restrict__ s = " << src << " + " << off << "L + b * " << sb << "L;\n"
      << "  float* __restrict__ d = " << out << " + b * " << R * C << "L;\n";
    if (sr == 1) {
      k << transpose_tile("float", R, C, sc, C, "s", "d", transpose_lanes(4, {R, C, sc, sb, off}));
    } else {
      k << "  const int t = threadIdx.x & 63, q = threadIdx.x >> 6;\n"
        << "  for (int r = q; r < 64; r += 4)\n"
        << "    if (r0 + r < " << R << "L && c0 + t < " << C << "L) d[(r0 + r) * " << C << "L + c0 + t] = s[(r0 + r) * " << sr
        << "L + (c0 + t) * " << sc << "L];\n";
    }
    k << "}\n";
    KernelStep ks;
    ks.source = k.str();
    ks.name = nm;
    ks.grid[0] = (uint32_t)(tr * tc);
    ks.grid[1] = (uint32_t)batch;
    ks.block[0] = 256;
    ks.klass = "pack";
    ks.label = "pack:slot" + std::to_string(slot);
    ks.algorithmic_bytes = 8.0 * (double)(batch * R * C);
    push(std::move(ks), w);
    return dst;
  }

  // Repacks the operands of a large f32 contraction whose layout the MFMA kernel does not take.
  void pack_f32_operands(GemmShape& gs) {
    auto ok4 = [](int64_t x) { return x % 4 == 0; };
    if (!(gs.a_k == 1 && ok4(gs.a_m) && ok4(gs.a_b) && ok4(gs.a.offset))) {
      const int s = pack_f32(gs.a.slot, gs.a.offset, gs.batch, gs.m, gs.k, gs.a_b, gs.a_m, gs.a_k);
      gs.a = View{s, 0, {}};
      gs.a_b = gs.m * gs.k;
      gs.a_m = gs.k;
      gs.a_k = 1;
      gs.ga_b = Group{{gs.batch}, {gs.a_b}};
      gs.ga_m = Group{{gs.m}, {gs.a_m}};
      gs.ga_k = Group{{gs.k}, {1}};
    }
    if (!(gs.b_n == 1 && ok4(gs.b_k) && ok4(gs.b_b) && ok4(gs.b.offset))) {
      const int s = pack_f32(gs.b.slot, gs.b.offset, gs.batch, gs.k, gs.n, gs.b_b, gs.b_k, gs.b_n);
      gs.b = View{s, 0, {}};
      gs.b_b = gs.k * gs.n;
      gs.b_k = gs.n;
      gs.b_n = 1;
      gs.gb_b = Group{{gs.batch}, {gs.b_b}};
      gs.gb_k = Group{{gs.k}, {gs.b_k}};
      gs.gb_n = Group{{gs.n}, {1}};
    }
  }

  // The MFMA templates take 16-bit operands whose K or M/N stride is 1, with 8-element aligned rows
  // (or, for operands whose groups span several axes, the direct-to-LDS kernel's layouts).
  bool gemm_eligible(const Op& op, GemmShape& gs) const {
    if (!opt_.allow_gemm) return false;
    DType d = op.result.dtype;
    if (d != DType::bf16 && d != DType::f16 && d != DType::f32) return false;
    if (!gemm_shape(op, gs)) return false;
    if (gs.m * gs.n * gs.k == 0) return false;
    if (gs.batch > 65535) return false;  // the batch index is gridDim.y, at most 65535 on gfx950
    if (d == DType::f32) {
      // The f32 MFMA kernel: 256 x 256 x 32 tiles, A K-contiguous and B N-contiguous with 16-byte
      // aligned rows. Exact tiles, or M / N off the tile grid (N a multiple of 4) when the problem is
      // large (2^27 multiply-adds and more); other f32 contractions keep runCpu's serial k order.
      // Large problems with another operand layout (an A stored M-contiguous, a B stored K-contiguous,
      // rows not 16-byte aligned) copy that operand into a contiguous temporary first (pack_f32).
      const bool exact = gs.m % 256 == 0 && gs.n % 256 == 0;
      const bool large = (double)gs.m * (double)gs.n * (double)gs.k * (double)gs.batch >= (double)(1ull << 27);
      if (gs.multi || !(exact || (large && gs.n % 4 == 0)) || gs.k % 32 != 0) return false;
      return f32_layout_ok(gs) || large;
    }
    if (gs.multi) {
      int dm, dn;
      bool akc, bkc;
      return dma_eligible(gs, dm, dn, akc, bkc);
    }
    auto ok8 = [](int64_t v) { return v % 8 == 0; };
    bool a_kc = gs.a_k == 1 && ok8(gs.k) && (gs.m == 1 || ok8(gs.a_m));
    bool a_mc = gs.a_m == 1 && ok8(gs.m) && (gs.k == 1 || ok8(gs.a_k));
    bool b_kc = gs.b_k == 1 && ok8(gs.k) && (gs.n == 1 || ok8(gs.b_n));
    bool b_nc = gs.b_n == 1 && ok8(gs.n) && (gs.k == 1 || ok8(gs.b_k));
    if (!(a_kc || a_mc) || !(b_kc || b_nc)) return false;
    if (!ok8(gs.a_b) || !ok8(gs.b_b) || !ok8(gs.a.offset) || !ok8(gs.b.offset)) return false;
    return true;
  }

  // Marks dot operands that are not plain views of a buffer: they are materialised first (by the
  // kernel that produces them, e.g. as a full-row output of a row kernel).
  void mark_gemm_operands() {
    for (uint32_t v = 0; v < g_.ops.size(); ++v) {
      const Op& op = g_.ops[v];
      if (!live_[v] || op.kind != Kind::dot_general || attn_.count(v)) continue;
      if (op.result.dtype != DType::bf16 && op.result.dtype != DType::f16 && op.result.dtype != DType::f32) continue;
      for (uint32_t a : op.args) {
        if (!view_chain_to_anchor(a)) needed_[a] = true;
      }
    }
  }

  // True when `v` is a (transpose / rename / broadcast) view of a parameter or an anchor value.
  bool view_chain_to_anchor(uint32_t v) const {
    const Op& op = g_.ops[v];
    switch (op.kind) {
      case Kind::transpose: case Kind::broadcast_in_dim: return view_chain_to_anchor(op.args[0]);
      case Kind::reshape: {
        const Type& it = g_.type(op.args[0]);
        if (it.rank() != op.result.rank()) return false;
        for (size_t k = 0; k < it.rank(); ++k)
          if (it.dims[k].extent != op.result.dims[k].extent) return false;
        return view_chain_to_anchor(op.args[0]);
      }
      case Kind::parameter: case Kind::dot_general: case Kind::reduce: case Kind::scatter_add: return true;
      default: return needed_[v];
    }
  }

  // ---- fused attention: dot(softmax_last(scale * dot(Q, K) [causal -inf mask]), V) ----
  //
  // The pattern is the one attention programs trace (a contraction, a scale by a splat constant, an
  // optional select of -inf where key > query, max, sub, exp, sum, div over the key axis, and the
  // contraction with V). Its intermediate values are absorbed when nothing else uses them; the
  // kernel computes the softmax in f32 online over key blocks (the accumulation order and the
  // rounding of the intermediate scores and probabilities differ from per-op 16-bit evaluation).
  struct Attn {
    uint32_t qk = 0;
    std::vector<uint32_t> inner;  // values computed only inside the fused kernel, in program order
    double scale = 1.0;
    bool causal = false;
  };
  std::map<uint32_t, Attn> attn_;

  // Value of a splat float constant, seen through broadcasts.
  bool splat_float(uint32_t v, double& out) const {
    const Op* op = &g_.ops[v];
    while (op->kind == Kind::broadcast_in_dim || op->kind == Kind::broadcast) op = &g_.ops[op->args[0]];
    if (op->kind != Kind::constant || !is_splat_constant(*op) || op->bytes.size() < 2) return false;
    const uint8_t* p = (const uint8_t*)op->bytes.data();
    switch (op->result.dtype) {
      case DType::f16: out = f16_bits_to_f32((uint16_t)(p[0] | (p[1] << 8))); return true;
      case DType::bf16: out = bf16_bits_to_f32((uint16_t)(p[0] | (p[1] << 8))); return true;
      case DType::f32: {
        if (op->bytes.size() < 4) return false;
        float f;
        std::memcpy(&f, p, 4);
        out = f;
        return true;
      }
      default: return false;
    }
  }

  // `v` = broadcast_in_dim(src) of a rank R-1 value back over the last axis of rank R.
  bool row_broadcast_of(uint32_t v, size_t R, uint32_t& src) const {
    const Op& op = g_.ops[v];
    if (op.kind != Kind::broadcast_in_dim || op.ints.size() != R - 1 || op.result.rank() != R) return false;
    for (size_t i = 0; i + 1 < R; ++i)
      if (op.ints[i] != (int64_t)i) return false;
    src = op.args[0];
    return true;
  }

  bool reduces_last(const Op& op, size_t R) const {
    return op.kind == Kind::reduce && op.ints.size() == 1 && op.ints[0] == (int64_t)R - 1 &&
           g_.type(op.args[0]).rank() == R;
  }

  // Which axis of its own type the integer value `v` equals the coordinate of (iota seen through
  // broadcast_in_dim), or -1.
  int index_axis(uint32_t v) const {
    const Op& op = g_.ops[v];
    if (op.kind == Kind::iota) return (int)op.axis;
    if (op.kind == Kind::broadcast_in_dim) {
      int a = index_axis(op.args[0]);
      return a < 0 ? -1 : (int)op.ints[(size_t)a];
    }
    return -1;
  }

  // `pred` (rank R) is true exactly where key index <= query index (query axis R-2, key axis R-1).
  bool causal_mask(uint32_t pred, size_t R) const {
    std::vector<int> map(R);
    for (size_t i = 0; i < R; ++i) map[i] = (int)i;
    uint32_t cur = pred;
    while (g_.ops[cur].kind == Kind::broadcast_in_dim) {
      const Op& b = g_.ops[cur];
      std::vector<int> nm(b.ints.size());
      for (size_t j = 0; j < b.ints.size(); ++j) nm[j] = map[(size_t)b.ints[j]];
      map = nm;
      cur = b.args[0];
    }
    const Op& c = g_.ops[cur];
    if (c.kind != Kind::compare) return false;
    int a = index_axis(c.args[0]), b = index_axis(c.args[1]);
    if (a < 0 || b < 0) return false;
    int sa = map[(size_t)a], sb = map[(size_t)b];
    const int q = (int)R - 2, k = (int)R - 1;
    Cmp cmp = (Cmp)c.code;
    return (cmp == Cmp::ge && sa == q && sb == k) || (cmp == Cmp::le && sa == k && sb == q);
  }

  bool match_attention(uint32_t pv, Attn& at) const {
    const Op& d = g_.ops[pv];
    const DType dt = d.result.dtype;
    if (d.kind != Kind::dot_general || (dt != DType::f16 && dt != DType::bf16 && dt != DType::f32)) return false;
    const uint32_t pdiv = d.args[0];
    const Op& dv = g_.ops[pdiv];
    const size_t R = dv.result.rank();
    if (R < 2 || dv.result.dtype != dt) return false;
    if (d.lhs_contract.size() != 1 || d.lhs_contract[0] != (int64_t)R - 1 || d.lhs_batch.size() != R - 2) return false;
    for (size_t i = 0; i + 2 < R; ++i)
      if (d.lhs_batch[i] != (int64_t)i) return false;
    if (dv.kind != Kind::binary || (Binary)dv.code != Binary::div) return false;
    const uint32_t e = dv.args[0];
    uint32_t sum, mx;
    double init;
    if (!row_broadcast_of(dv.args[1], R, sum)) return false;
    const Op& so = g_.ops[sum];
    if (!reduces_last(so, R) || (Reducer)so.code != Reducer::sum || so.args[0] != e) return false;
    if (!splat_float(so.args[1], init) || init != 0.0) return false;
    const Op& eo = g_.ops[e];
    if (eo.kind != Kind::unary || (Unary)eo.code != Unary::exp) return false;
    const uint32_t sub = eo.args[0];
    const Op& subo = g_.ops[sub];
    if (subo.kind != Kind::binary || (Binary)subo.code != Binary::sub) return false;
    if (!row_broadcast_of(subo.args[1], R, mx)) return false;
    const uint32_t s = subo.args[0];
    const Op& mo = g_.ops[mx];
    if (!reduces_last(mo, R) || (Reducer)mo.code != Reducer::max || mo.args[0] != s) return false;
    if (!splat_float(mo.args[1], init) || !(std::isinf(init) && init < 0)) return false;
    std::vector<uint32_t> inner = {pdiv, dv.args[1], sum, e, sub, subo.args[1], mx};
    uint32_t x = s;
    at.causal = false;
    at.scale = 1.0;
    if (g_.ops[x].kind == Kind::select) {
      const Op& sel = g_.ops[x];
      double f;
      if (!splat_float(sel.args[2], f) || !(std::isinf(f) && f < 0) || !causal_mask(sel.args[0], R)) return false;
      at.causal = true;
      inner.push_back(x);
      x = sel.args[1];
    }
    // Scale steps: multiplications or divisions by splat constants.
    while (g_.ops[x].kind == Kind::binary) {
      const Op& b = g_.ops[x];
      inner.push_back(x);
      double c;
      if ((Binary)b.code == Binary::mul && splat_float(b.args[1], c)) {
        at.scale *= c;
        x = b.args[0];
      } else if ((Binary)b.code == Binary::mul && splat_float(b.args[0], c)) {
        at.scale *= c;
        x = b.args[1];
      } else if ((Binary)b.code == Binary::div && splat_float(b.args[1], c)) {
        at.scale /= c;
        x = b.args[0];
      } else {
        return false;
      }
    }
    if (!(at.scale > 0) || !std::isfinite(at.scale)) return false;
    const Op& qk = g_.ops[x];
    if (qk.kind != Kind::dot_general || qk.result.dtype != dt || qk.result.dims != dv.result.dims) return false;
    if (qk.lhs_contract.size() != 1 || qk.rhs_contract.size() != 1 || qk.lhs_batch.size() != R - 2) return false;
    inner.push_back(x);
    std::sort(inner.begin(), inner.end());
    inner.erase(std::unique(inner.begin(), inner.end()), inner.end());
    // Nothing outside the pattern may read an absorbed value.
    for (uint32_t u = 0; u < g_.ops.size(); ++u) {
      if (!live_[u] || u == pv || std::binary_search(inner.begin(), inner.end(), u)) continue;
      for (uint32_t a : g_.ops[u].args)
        if (std::binary_search(inner.begin(), inner.end(), a)) return false;
    }
    for (uint32_t o : g_.outputs)
      if (std::binary_search(inner.begin(), inner.end(), o)) return false;
    at.qk = x;
    at.inner = inner;
    return true;
  }

  void match_attentions() {
    if (!opt_.allow_gemm) return;
    for (uint32_t v = 0; v < g_.ops.size(); ++v) {
      if (!live_[v] || g_.ops[v].kind != Kind::dot_general) continue;
      Attn at;
      if (!match_attention(v, at)) continue;
      for (uint32_t u : at.inner) done_[u] = true;
      attn_[v] = at;
    }
  }

  struct AttnLayout {
    int64_t sq = 0, sk = 0, nb = 1, q_s = 0, k_s = 0, v_s = 0, hd = 0;
    std::vector<int64_t> extents, q_b, k_b, v_b;  // batch axes: extents and per-operand strides
    View q, k, v;
  };

  static int free_axis(size_t rank, const std::vector<int64_t>& batch, const std::vector<int64_t>& contract) {
    int f = -1;
    for (size_t i = 0; i < rank; ++i) {
      if (std::find(batch.begin(), batch.end(), (int64_t)i) != batch.end()) continue;
      if (std::find(contract.begin(), contract.end(), (int64_t)i) != contract.end()) continue;
      if (f >= 0) return -2;
      f = (int)i;
    }
    return f;
  }

  bool attention_layout(uint32_t pv, const Attn& at, AttnLayout& L) const {
    const Op& d = g_.ops[pv];
    const Op& qk = g_.ops[at.qk];
    if (!resolve_view(qk.args[0], L.q) || !resolve_view(qk.args[1], L.k) || !resolve_view(d.args[1], L.v)) return false;
    const Type& qt = g_.type(qk.args[0]);
    const Type& kt = g_.type(qk.args[1]);
    const Type& vt = g_.type(d.args[1]);
    const int qf = free_axis(qt.rank(), qk.lhs_batch, qk.lhs_contract);
    const int kf = free_axis(kt.rank(), qk.rhs_batch, qk.rhs_contract);
    const int vf = free_axis(vt.rank(), d.rhs_batch, d.rhs_contract);
    if (qf < 0 || kf < 0 || vf < 0 || d.rhs_contract.size() != 1) return false;
    const size_t qc = (size_t)qk.lhs_contract[0], kc = (size_t)qk.rhs_contract[0], vc = (size_t)d.rhs_contract[0];
    // Head dimension (Q.K contraction and V's free axis, unit stride): 64, 128 or 256 for 16-bit
    // operands (attn::flash), 64 for f32 (attn::flash_f32, the reference's flash pattern).
    const bool f32 = d.result.dtype == DType::f32;
    L.hd = qt.dims[qc].extent;
    if (f32 ? L.hd != 64 : (L.hd != 64 && L.hd != 128 && L.hd != 256)) return false;
    if (kt.dims[kc].extent != L.hd || vt.dims[(size_t)vf].extent != L.hd) return false;
    if (L.q.strides[qc] != 1 || L.k.strides[kc] != 1 || L.v.strides[(size_t)vf] != 1) return false;
    L.sq = qt.dims[(size_t)qf].extent;
    L.sk = kt.dims[(size_t)kf].extent;
    // 32 queries per wave and key blocks of 32 (both kernels)
    if (vt.dims[vc].extent != L.sk || L.sq % 32 != 0 || L.sk % 32 != 0 || L.sq == 0 || L.sk == 0) return false;
    L.q_s = L.q.strides[(size_t)qf];
    L.k_s = L.k.strides[(size_t)kf];
    L.v_s = L.v.strides[vc];
    // 16-byte aligned rows and batch offsets (8 16-bit or 4 f32 elements)
    const int64_t al = f32 ? 4 : 8;
    auto ok8 = [al](int64_t x) { return x % al == 0; };
    if (!ok8(L.q_s) || !ok8(L.k_s) || !ok8(L.v_s) || !ok8(L.q.offset) || !ok8(L.k.offset) || !ok8(L.v.offset)) return false;
    for (size_t i = 0; i < qk.lhs_batch.size(); ++i) {
      const int64_t e = qt.dims[(size_t)qk.lhs_batch[i]].extent;
      if (kt.dims[(size_t)qk.rhs_batch[i]].extent != e || vt.dims[(size_t)d.rhs_batch[i]].extent != e) return false;
      L.extents.push_back(e);
      L.q_b.push_back(L.q.strides[(size_t)qk.lhs_batch[i]]);
      L.k_b.push_back(L.k.strides[(size_t)qk.rhs_batch[i]]);
      L.v_b.push_back(L.v.strides[(size_t)d.rhs_batch[i]]);
      if (!ok8(L.q_b.back()) || !ok8(L.k_b.back()) || !ok8(L.v_b.back())) return false;
      L.nb *= e;
    }
    return L.nb > 0;
  }

  // Element offset of flattened (row-major) batch index b for one operand.
  static std::string batch_offset(const std::vector<int64_t>& extents, const std::vector<int64_t>& strides,
                                  int64_t offset) {
    std::ostringstream s;
    s << offset << "L";
    int64_t inner = 1;
    for (size_t i = extents.size(); i-- > 0;) {
      if (extents[i] != 1 && strides[i] != 0) {
        s << " + ((b / " << inner << "L) % " << extents[i] << "L) * " << strides[i] << "L";
      }
      inner *= extents[i];
    }
    return s.str();
  }

  void attention(uint32_t pv, const Attn& at, const AttnLayout& L) {
    const Op& d = g_.ops[pv];
    const DType dt = d.result.dtype;
    if (dt == DType::f32) {
      attention_f32(pv, at, L);
      return;
    }
    int out = slots_.slot_of[pv] >= 0 ? slots_.slot_of[pv] : temp_slot(pv);
    // Waves per workgroup (32 queries each): eight (two per SIMD) when the queries divide, else the
    // largest count that does, with two or more workgroups per CU; every wave's share of a K / V tile
    // (HD / 16 load instructions) must be whole. Head dimension 256 takes at most four (one wave per
    // SIMD: its O and Q^T alone fill 192 registers, and its K / V stages 128 KiB of LDS).
    int waves = 1;
    for (int w : {8, 4, 2}) {
      if (L.hd == 256 && w > 4) continue;
      if (L.sq % (32 * w) == 0 && (L.hd / 16) % w == 0) {
        waves = w;
        break;
      }
    }
    KernelWriter w(g_, slots_, "i64_t");
    std::string q = w.arg(L.q.slot, false), k = w.arg(L.k.slot, false), v = w.arg(L.v.slot, false),
                o = w.arg(out, true);
    std::string nm = name("attention", pv);
    char sl[64];
    std::snprintf(sl, sizeof sl, "%af", (double)(float)(at.scale * 1.4426950408889634));
    std::ostringstream src;
    src << kMfmaVgprForm << "#include \"gemm\"\n#include \"attention\"\n";
    src << "struct Cfg_" << nm << " {\n"
        << "  static constexpr int DT = " << (dt == DType::bf16 ? 0 : 1) << ", HD = " << L.hd << ", WAVES = " << waves
        << ";\n"
        << "  static constexpr long SQ = " << L.sq << ", SK = " << L.sk << ", NB = " << L.nb << ";\n"
        << "  static constexpr long Q_S = " << L.q_s << ", K_S = " << L.k_s << ", V_S = " << L.v_s << ";\n"
        << "  static constexpr bool CAUSAL = " << (at.causal ? "true" : "false") << ";\n"
        << "  static constexpr float SL = " << sl << ";\n"
        << "  static __device__ __forceinline__ long q_off(long b) { return " << batch_offset(L.extents, L.q_b, L.q.offset)
        << "; }\n"
        << "  static __device__ __forceinline__ long k_off(long b) { return " << batch_offset(L.extents, L.k_b, L.k.offset)
        << "; }\n"
        << "  static __device__ __forceinline__ long v_off(long b) { return " << batch_offset(L.extents, L.v_b, L.v.offset)
        << "; }\n};\n";
    // One parameter per distinct buffer (Q, K and V may share one).
    std::string params;
    for (const std::string& x : {q, k, v}) {
      if (params.find("* __restrict__ " + x + ",") != std::string::npos) continue;
      params += "const u16_t* __restrict__ " + x + ", ";
    }
    params += "u16_t* __restrict__ " + o;
    src << "extern \"C\" __global__ void __launch_bounds__(" << 64 * waves << ") " << nm << "(" << params
        << ") {\n  accy::attn::flash<Cfg_" << nm << ">(" << q << ", " << k << ", " << v << ", " << o << ");\n}\n";
    KernelStep ks;
    ks.source = src.str();
    ks.name = nm;
    // Causal with an even number of query blocks: two complementary blocks per workgroup
    // (attn::blocks_per_group), so every workgroup streams the same number of keys.
    const int64_t nqb = L.sq / (32 * waves);
    const int64_t pair = at.causal && nqb % 2 == 0 ? 2 : 1;
    ks.grid[0] = (uint32_t)(L.nb * nqb / pair);
    ks.block[0] = 64 * waves;  // one wave per 32 queries
    ks.klass = "attention";
    ks.label = "attention:%" + std::to_string(pv);
    ks.algorithmic_flops = 4.0 * (double)L.nb * attention_pairs(at, L) * (double)L.hd;
    push(std::move(ks), w);
    finish(pv);
  }

  // Score pairs the kernel computes: all of them, or those with key <= query under the causal mask.
  static double attention_pairs(const Attn& at, const AttnLayout& L) {
    double pairs = (double)L.sq * (double)L.sk;
    if (at.causal) {
      const double n = (double)std::min(L.sq, L.sk);
      pairs = n * (n + 1) / 2 + (L.sq > L.sk ? (double)(L.sq - L.sk) * (double)L.sk : 0.0);
    }
    return pairs;
  }

  // f32 attention of head dimension 64 (attn::flash_f32): 32 queries per wave.
  void attention_f32(uint32_t pv, const Attn& at, const AttnLayout& L) {
    int out = slots_.slot_of[pv] >= 0 ? slots_.slot_of[pv] : temp_slot(pv);
    const int waves = L.sq % 128 == 0 ? 4 : (L.sq % 64 == 0 ? 2 : 1);
    KernelWriter w(g_, slots_, "i64_t");
    std::string q = w.arg(L.q.slot, false), k = w.arg(L.k.slot, false), v = w.arg(L.v.slot, false),
                o = w.arg(out, true);
    std::string nm = name("attention", pv);
    char sl[64];
    std::snprintf(sl, sizeof sl, "%af", (double)(float)(at.scale * 1.4426950408889634));
    std::ostringstream src;
    src << "#include \"gemm\"\n#include \"attention\"\n";
    src << "struct Cfg_" << nm << " {\n"
        << "  static constexpr int WAVES = " << waves << ";\n"
        << "  static constexpr long SQ = " << L.sq << ", SK = " << L.sk << ", NB = " << L.nb << ";\n"
        << "  static constexpr long Q_S = " << L.q_s << ", K_S = " << L.k_s << ", V_S = " << L.v_s << ";\n"
        << "  static constexpr bool CAUSAL = " << (at.causal ? "true" : "false") << ";\n"
        << "  static constexpr float SL = " << sl << ";\n"
        << "  static __device__ __forceinline__ long q_off(long b) { return " << batch_offset(L.extents, L.q_b, L.q.offset)
        << "; }\n"
        << "  static __device__ __forceinline__ long k_off(long b) { return " << batch_offset(L.extents, L.k_b, L.k.offset)
        << "; }\n"
        << "  static __device__ __forceinline__ long v_off(long b) { return " << batch_offset(L.extents, L.v_b, L.v.offset)
        << "; }\n};\n";
    std::string params;
    for (const std::string& x : {q, k, v}) {
      if (params.find("* __restrict__ " + x + ",") != std::string::npos) continue;
      params += "const float* __restrict__ " + x + ", ";
    }
    params += "float* __restrict__ " + o;
    src << "extern \"C\" __global__ void __launch_bounds__(" << 64 * waves << ") " << nm << "(" << params
        << ") {\n  accy::attn::flash_f32<Cfg_" << nm << ">(" << q << ", " << k << ", " << v << ", " << o << ");\n}\n";
    KernelStep ks;
    ks.source = src.str();
    ks.name = nm;
    ks.grid[0] = (uint32_t)(L.nb * (L.sq / (32 * waves)));
    ks.block[0] = 64 * waves;
    ks.klass = "attention";
    ks.label = "attention:%" + std::to_string(pv);
    ks.algorithmic_flops = 4.0 * (double)L.nb * attention_pairs(at, L) * (double)L.hd;
    push(std::move(ks), w);
    finish(pv);
  }


  void dot(uint32_t v) {
    const Op& op = g_.ops[v];
    auto fused = attn_.find(v);
    if (fused != attn_.end()) {
      AttnLayout L;
      if (attention_layout(v, fused->second, L)) {
        attention(v, fused->second, L);
        return;
      }
      // Operands the kernel cannot address: compute the absorbed values after all, in order.
      needed_[op.args[0]] = true;
      std::vector<uint32_t> inner = fused->second.inner;
      attn_.erase(fused);
      for (uint32_t u : inner) done_[u] = false;
      for (uint32_t u : inner)
        if (!done_[u]) process(u);
    }
    GemmShape gs;
    if (gemm_eligible(op, gs)) {
      if (op.result.dtype == DType::f32 && !f32_layout_ok(gs)) pack_f32_operands(gs);
      std::vector<std::pair<uint32_t, GemmShape>> group;
      if (gemm_siblings(v, gs, group)) {
        gemm_group(group);
        return;
      }
      gemm(v, gs);
      return;
    }
    dot_serial(v);
  }

  // ---- grouped contractions: several contractions of one activation in one launch ----
  //
  // dot_general v and the later, not yet planned contractions u with the same A view (same buffer,
  // offset and layout), the same extents and the same B layout, whose B operands are already
  // available and whose results are plain stores (no fused epilogue, no attention): the projections
  // of one normalised activation. They run as one direct-to-LDS launch of G x tiles workgroups
  // (mma16_dma_group), so the machine fills and drains once instead of G times. Every output keeps
  // its own k order and accumulation, so the results are those of separate launches bit for bit.
  static bool same_group(const Group& x, const Group& y) { return x.ext == y.ext && x.str == y.str; }

  bool plain_store(uint32_t u) const {
    uint32_t t;
    return attn_.find(u) == attn_.end() && !epilogue_target(u, t);
  }

  bool gemm_siblings(uint32_t v, const GemmShape& gs, std::vector<std::pair<uint32_t, GemmShape>>& group) const {
    const Op& op = g_.ops[v];
    const DType d = op.result.dtype;
    if (op.kind != Kind::dot_general || (d != DType::bf16 && d != DType::f16) || gs.multi) return false;
    if (gs.m % 256 != 0 || gs.n % 256 != 0 || std::getenv("ACCY_GEMM_NO_GROUP")) return false;
    int dm = 0, dn = 0;
    bool akc = gs.a_k == 1, bkc = gs.b_k == 1;
    if (!dma_eligible(gs, dm, dn, akc, bkc) || dm != 256 || dn != 256 || !plain_store(v)) return false;
    group.assign(1, {v, gs});
    constexpr size_t kMaxGroup = 4;
    for (uint32_t u = v + 1; u < g_.ops.size() && group.size() < kMaxGroup; ++u) {
      const Op& uo = g_.ops[u];
      if (!live_[u] || done_[u] || uo.kind != Kind::dot_general || uo.args[0] != op.args[0] || uo.result.dtype != d)
        continue;
      GemmShape gu;
      if (!gemm_eligible(uo, gu) || gu.multi || !plain_store(u)) continue;
      if (gu.batch != gs.batch || gu.m != gs.m || gu.n != gs.n || gu.k != gs.k) continue;
      if (gu.a.slot != gs.a.slot || gu.a.offset != gs.a.offset || gu.a_b != gs.a_b || gu.a_m != gs.a_m ||
          gu.a_k != gs.a_k || gu.b_b != gs.b_b || gu.b_k != gs.b_k || gu.b_n != gs.b_n)
        continue;
      if (!same_group(gu.ga_b, gs.ga_b) || !same_group(gu.ga_m, gs.ga_m) || !same_group(gu.ga_k, gs.ga_k) ||
          !same_group(gu.gb_b, gs.gb_b) || !same_group(gu.gb_k, gs.gb_k) || !same_group(gu.gb_n, gs.gb_n))
        continue;
      int um = 0, un = 0;
      bool uak = gu.a_k == 1, ubk = gu.b_k == 1;
      if (!dma_eligible(gu, um, un, uak, ubk) || um != dm || un != dn || uak != akc || ubk != bkc) continue;
      group.push_back({u, gu});
    }
    return group.size() > 1;
  }

  void gemm_group(const std::vector<std::pair<uint32_t, GemmShape>>& group) {
    const uint32_t v = group[0].first;
    const GemmShape& gs = group[0].second;
    const DType d = g_.ops[v].result.dtype;
    const size_t G = group.size();
    KernelWriter w(g_, slots_, "i64_t");
    const std::string a = w.arg(gs.a.slot, false);
    std::vector<std::string> bs;
    std::ostringstream cases;
    const std::string cidx = "b * " + std::to_string(gs.m * gs.n) + "L + m * " + std::to_string(gs.n) + "L + n";
    std::string nm = name("gemm", v), label = "gemm:%" + std::to_string(v);
    for (size_t i = 0; i < G; ++i) {
      const uint32_t u = group[i].first;
      bs.push_back(w.arg(group[i].second.b.slot, false) + " + " + std::to_string(group[i].second.b.offset) + "L");
      const int out = slots_.slot_of[u] >= 0 ? slots_.slot_of[u] : temp_slot(u);
      cases << "      case " << i << ": " << w.store(out, cidx, d, "v") << " break;\n";
      if (i) label += "&%" + std::to_string(u);
    }
    std::ostringstream members, inits;
    {
      std::string pl = w.params();
      size_t start = 0;
      while (start < pl.size()) {
        size_t comma = pl.find(", ", start);
        std::string decl = pl.substr(start, comma == std::string::npos ? std::string::npos : comma - start);
        members << "  " << decl << ";\n";
        size_t sp = decl.rfind(' ');
        inits << (inits.tellp() > 0 ? ", " : "") << decl.substr(sp + 1);
        if (comma == std::string::npos) break;
        start = comma + 2;
      }
    }
    std::ostringstream src;
    src << "#include \"gemm\"\n";
    src << "struct Epi_" << nm << " {\n" << members.str()
        << "  __device__ __forceinline__ void operator()(int g, long b, long m, long n, float v) const {\n"
        << "    switch (g) {\n" << cases.str() << "    }\n  }\n};\n";
    src << "struct Cfg_" << nm << " {\n"
        << "  static constexpr int DT = " << (d == DType::bf16 ? 0 : 1) << ";\n"
        << "  static constexpr long M = " << gs.m << ", N = " << gs.n << ", K = " << gs.k << ";\n"
        << "  static constexpr long A_B = " << gs.a_b << ", A_M = " << gs.a_m << ", A_K = " << gs.a_k << ";\n"
        << "  static constexpr long B_B = " << gs.b_b << ", B_K = " << gs.b_k << ", B_N = " << gs.b_n << ";\n"
        << "  static constexpr bool A_KC = " << (gs.a_k == 1 ? "true" : "false")
        << ", B_KC = " << (gs.b_k == 1 ? "true" : "false") << ";\n"
        << gs.ga_b.fn("a_b") << gs.ga_m.fn("a_m") << gs.ga_k.fn("a_k") << gs.gb_b.fn("b_b") << gs.gb_k.fn("b_k")
        << gs.gb_n.fn("b_n") << "  static constexpr int BM = 256, BN = 256, STAGES = 4;\n};\n";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << nm << "(" << w.params() << ") {\n"
        << "  const u16_t* const bs[" << G << "] = {";
    for (size_t i = 0; i < G; ++i) src << (i ? ", " : "") << bs[i];
    src << "};\n  accy::gemm::mma16_dma_group<Cfg_" << nm << ", " << G << ">(" << a << " + " << gs.a.offset
        << "L, bs, Epi_" << nm << "{" << inits.str() << "});\n}\n";
    KernelStep k;
    k.source = src.str();
    k.name = nm;
    k.grid[0] = (uint32_t)(G * (size_t)((gs.m / 256) * (gs.n / 256)));
    k.grid[1] = (uint32_t)gs.batch;
    k.block[0] = 256;
    k.klass = "gemm";
    k.label = label;
    k.algorithmic_flops = 2.0 * (double)G * (double)gs.batch * (double)gs.m * (double)gs.n * (double)gs.k;
    push(std::move(k), w);
    for (const auto& member : group) finish(member.first);
  }

  // Output layout of a contraction result: strides of the flattened batch, m and n groups.
  struct OutStrides {
    int64_t b = 0, m = 0, n = 1;
  };

  void gemm(uint32_t v, const GemmShape& gs) {
    OutStrides os;
    os.b = gs.m * gs.n;
    os.m = gs.n;
    os.n = 1;
    gemm(v, gs, os);
  }

  // ---- contraction epilogues ----
  //
  // When the contraction's value v is not itself materialised and every use of it runs through
  // elementwise operations of v's shape into exactly one materialised value u (an activation, a
  // residual add), the kernel's epilogue computes u from the accumulator and stores u: v never
  // travels through HBM. Other operands of u's expression are read at the same index.
  bool epilogue_target(uint32_t v, uint32_t& target) const {
    if (needed_[v] || slots_.slot_of[v] >= 0) return false;
    const Type& vt = g_.type(v);
    std::vector<std::vector<uint32_t>> users(g_.ops.size());
    for (uint32_t u = v + 1; u < g_.ops.size(); ++u)
      if (live_[u] && !done_[u])
        for (uint32_t a : g_.ops[u].args) users[a].push_back(u);
    std::set<uint32_t> region = {v}, targets;
    std::vector<uint32_t> stack = {v};
    while (!stack.empty()) {
      uint32_t x = stack.back();
      stack.pop_back();
      for (uint32_t u : users[x]) {
        const Op& uo = g_.ops[u];
        bool elementwise = uo.kind == Kind::unary || uo.kind == Kind::binary || uo.kind == Kind::select ||
                           uo.kind == Kind::compare;
        if (!elementwise || !(uo.result.dims == vt.dims)) return false;
        if (needed_[u]) {
          targets.insert(u);
        } else if (!region.count(u)) {
          region.insert(u);
          stack.push_back(u);
        }
      }
    }
    if (targets.size() != 1) return false;
    const uint32_t u = *targets.begin();
    if (done_[u]) return false;
    target = u;
    return true;
  }

  // A fused epilogue worth a lookup table: contraction and result both 16-bit, and the result a chain
  // of at least six elementwise operations whose leaves are the contraction value and splat float
  // constants only (no other tensor, no index), so it is a function of the rounded contraction value.
  bool lut_epilogue(uint32_t v, uint32_t target, DType d, DType td) const {
    auto b16 = [](DType t) { return t == DType::bf16 || t == DType::f16; };
    if (!b16(d) || !b16(td) || target == v || std::getenv("ACCY_GEMM_NO_LUT")) return false;
    std::set<uint32_t> seen;
    int ops = 0;
    std::function<bool(uint32_t)> ok = [&](uint32_t x) -> bool {
      if (x == v || seen.count(x)) return true;
      double c;
      if (splat_float(x, c)) return true;
      const Op& o = g_.ops[x];
      const bool ew = o.kind == Kind::unary || o.kind == Kind::binary || o.kind == Kind::select ||
                      o.kind == Kind::compare;
      if (!ew) return false;
      seen.insert(x);
      ++ops;
      for (uint32_t a : o.args)
        if (!ok(a)) return false;
      return true;
    };
    return ok(target) && ops >= 6;
  }

  // Writes the contraction described by gs into the slot of value v (laid out per os), or, with a
  // fused epilogue, the value that the elementwise region after v materialises.
  void gemm(uint32_t v, const GemmShape& gs, const OutStrides& os) {
    const Op& op = g_.ops[v];
    DType d = op.result.dtype;
    const std::string cidx = "b * " + std::to_string(os.b) + "L + m * " + std::to_string(os.m) + "L + n * " +
                             std::to_string(os.n) + "L";
    std::string nm = name("gemm", v);
    uint32_t target = v;
    std::unique_ptr<KernelWriter> w;
    std::ostringstream epi;
    std::string table_members;  // a lookup-table epilogue's interface (gemm.h HasTable)
    // The fused epilogue (dot_general results only: os is their row-major layout).
    const bool rowmajor = os.b == gs.m * gs.n && os.m == gs.n && os.n == 1;
    if (op.kind == Kind::dot_general && rowmajor && epilogue_target(v, target)) {
      try {
        w.reset(new KernelWriter(g_, slots_, "i64_t"));
        w->arg(gs.a.slot, false);
        w->arg(gs.b.slot, false);
        const Type& rt = op.result;
        const size_t nb = op.lhs_batch.size();
        const size_t nlf = rt.rank() - nb - (g_.type(op.args[1]).rank() - op.rhs_batch.size() - op.rhs_contract.size());
        std::vector<Dim> bd(rt.dims.begin(), rt.dims.begin() + (long)nb);
        std::vector<Dim> md(rt.dims.begin() + (long)nb, rt.dims.begin() + (long)(nb + nlf));
        std::vector<Dim> ndims(rt.dims.begin() + (long)(nb + nlf), rt.dims.end());
        std::vector<std::string> coords;
        for (auto& c : delinearize("b", bd)) coords.push_back(c);
        for (auto& c : delinearize("m", md)) coords.push_back(c);
        for (auto& c : delinearize("n", ndims)) coords.push_back(c);
        Scope sc(epi, "    ");
        w->provide = [&](uint32_t vid, const std::vector<std::string>& c, std::string& out) -> bool {
          if (vid != v) return false;
          if (c != coords) throw NotFusable("contraction value read at another index");
          out = "vv";
          return true;
        };
        const DType td = g_.type(target).dtype;
        if (lut_epilogue(v, target, d, td)) {
          // A 16-bit epilogue that is a function of the rounded contraction value alone: a table
          // kernel evaluates the same generated expression for all 65536 bit patterns, and the
          // contraction's epilogue is one lookup per element (bit-identical by construction).
          const int tslot = slots_.add(SlotInfo::Temp, -1, td, 65536u * 2u);
          KernelWriter tw(g_, slots_, "i64_t");
          tw.arg(tslot, true);
          std::ostringstream tk;
          Scope tsc(tk, "  ");
          tw.provide = [&](uint32_t vid, const std::vector<std::string>&, std::string& out) -> bool {
            if (vid != v) return false;
            out = "vv";
            return true;
          };
          const std::string tx = tw.value(target, coords, tsc);
          const std::string tnm = name("lut", target);
          std::ostringstream tsrc;
          tsrc << "extern \"C\" __global__ void __launch_bounds__(256) " << tnm << "(" << tw.params() << ") {\n"
               << "  const int i = (int)(blockIdx.x * 256 + threadIdx.x);\n"
               << "  const float vv = " << (d == DType::bf16 ? "accy::bf16_to_f32" : "accy::f16_to_f32") << "((u16_t)i);\n"
               << tk.str() << "  " << tw.store(tslot, "i", td, tx) << "\n}\n";
          KernelStep ts;
          ts.source = tsrc.str();
          ts.name = tnm;
          ts.grid[0] = 256;
          ts.block[0] = 256;
          ts.klass = "lut";
          ts.label = "lut:%" + std::to_string(target);
          ts.once = true;
          const std::string tab = w->arg(tslot, false);
          int out = slots_.slot_of[target] >= 0 ? slots_.slot_of[target] : temp_slot(target);
          const std::string dst = w->arg(out, true);
          const std::string idx = d == DType::bf16 ? "accy::f32_to_bf16(v)" : "accy::f32_to_f16(v)";
          epi << "    " << dst << "[" << cidx << "] = " << tab << "[" << idx << "];\n";
          table_members = "  static constexpr bool kTable = true;\n"
                          "  __device__ __forceinline__ const u16_t* table() const { return " + tab + "; }\n"
                          "  static __device__ __forceinline__ u16_t index(float v) { return " + idx + "; }\n"
                          "  __device__ __forceinline__ void put(long b, long m, long n, u16_t bits) const { " +
                          dst + "[" + cidx + "] = bits; }\n";
          push(std::move(ts), tw);
        } else {
          std::string x = w->value(target, coords, sc);
          int out = slots_.slot_of[target] >= 0 ? slots_.slot_of[target] : temp_slot(target);
          epi << sc.indent << w->store(out, cidx, td, x) << "\n";
        }
      } catch (const NotFusable&) {
        target = v;
        w.reset();
        epi.str("");
      }
    }
    if (!w) {
      w.reset(new KernelWriter(g_, slots_, "i64_t"));
      w->arg(gs.a.slot, false);
      w->arg(gs.b.slot, false);
      int out = slots_.slot_of[v] >= 0 ? slots_.slot_of[v] : temp_slot(v);
      epi << "    " << w->store(out, cidx, d, "v") << "\n";
    }
    const std::string a = w->arg(gs.a.slot, false), b = w->arg(gs.b.slot, false);
    // Epilogue functor: every buffer of the kernel as a member named like the kernel parameter.
    std::ostringstream members, inits;
    {
      std::string pl = w->params();
      size_t start = 0;
      while (start < pl.size()) {
        size_t comma = pl.find(", ", start);
        std::string decl = pl.substr(start, comma == std::string::npos ? std::string::npos : comma - start);
        members << "  " << decl << ";\n";
        size_t sp = decl.rfind(' ');
        inits << (inits.tellp() > 0 ? ", " : "") << decl.substr(sp + 1);
        if (comma == std::string::npos) break;
        start = comma + 2;
      }
    }
    std::ostringstream src;
    KernelStep k;
    src << "#include \"gemm\"\n";
    src << "struct Epi_" << nm << " {\n" << members.str()
        << table_members
        << "  __device__ __forceinline__ void operator()(long b, long m, long n, float v) const {\n"
        << (target != v && table_members.empty() ? "    const float vv = " + round_to(d, "v") + ";\n" : "") << epi.str()
        << "  }\n};\n";
    if (d == DType::f32) {
      // f32 on v_mfma_f32_32x32x2_f32: exact 256 x 256 x 32 tiles (gemm_eligible checked the layout).
      src << "struct Cfg_" << nm << " {\n"
          << "  static constexpr long M = " << gs.m << ", N = " << gs.n << ", K = " << gs.k << ";\n"
          << gs.ga_b.fn("a_b") << gs.ga_m.fn("a_m") << gs.ga_k.fn("a_k") << gs.gb_b.fn("b_b") << gs.gb_k.fn("b_k")
          << gs.gb_n.fn("b_n") << "};\n";
      src << "extern \"C\" __global__ void __launch_bounds__(256) " << nm << "(" << w->params() << ") {\n"
          << "  accy::gemm::mma32f<Cfg_" << nm << ">(" << a << " + " << gs.a.offset << "L, " << b << " + "
          << gs.b.offset << "L, Epi_" << nm << "{" << inits.str() << "});\n}\n";
      k.grid[0] = (uint32_t)(((gs.m + 255) / 256) * ((gs.n + 255) / 256));
      k.block[0] = 256;
    } else {
      // 256 x 256 x 64 tiles; the wave grid (4 x 2 waves of 64 x 128, or 2 x 2 waves of 128 x 128)
      // can be overridden with ACCY_GEMM_WAVES=MxN for tuning.
      const int BM = 256, BN = 256, BK = 64;
      int WM = 2, WN = 2;
      if (const char* e = std::getenv("ACCY_GEMM_WAVES")) {
        int mm = 0, nn = 0;
        if (std::sscanf(e, "%dx%d", &mm, &nn) == 2 && (mm == 2 || mm == 4) && (nn == 2 || nn == 4) && mm * nn <= 8) {
          WM = mm;
          WN = nn;
        }
      }
      // Direct-to-LDS pipeline when the tiles divide the problem exactly (every row start 16-byte
      // aligned); otherwise the register-staged kernel, which guards edges (single strides only).
      int dm = 0, dn = 0;
      bool akc = gs.a_k == 1, bkc = gs.b_k == 1;
      bool dma = dma_eligible(gs, dm, dn, akc, bkc);
      src << "struct Cfg_" << nm << " {\n"
          << "  static constexpr int DT = " << (d == DType::bf16 ? 0 : 1) << ";\n"
          << "  static constexpr long M = " << gs.m << ", N = " << gs.n << ", K = " << gs.k << ";\n"
          << "  static constexpr long A_B = " << gs.a_b << ", A_M = " << gs.a_m << ", A_K = " << gs.a_k << ";\n"
          << "  static constexpr long B_B = " << gs.b_b << ", B_K = " << gs.b_k << ", B_N = " << gs.b_n << ";\n"
          << "  static constexpr bool A_KC = " << (akc ? "true" : "false") << ", B_KC = " << (bkc ? "true" : "false")
          << ";\n"
          << gs.ga_b.fn("a_b") << gs.ga_m.fn("a_m") << gs.ga_k.fn("a_k") << gs.gb_b.fn("b_b") << gs.gb_k.fn("b_k")
          << gs.gb_n.fn("b_n");
      // Launch candidates of the direct-to-LDS kernel (bit-identical results: every output keeps its
      // k order): the N tile, 256 (4 stages, one workgroup per CU, 128 KiB of LDS), then 128 where
      // B's layout allows it. (256 x 128 with 3 stages and two workgroups per CU was measured too:
      // its LDS traffic per MFMA is half as large again as the 256 x 256 tile's, and it ran 20-40 %
      // slower on every benchmark contraction.) The source carries a placeholder until the candidate
      // is chosen.
      std::vector<int> n_tiles{dn};
      if (dma && dn == 256) {
        bool kc2 = bkc;
        if (dma_operand(gs.gb_n, gs.gb_k, gs.gb_b, gs.b.offset, 128, kc2) && kc2 == bkc) n_tiles.push_back(128);
      }
      const bool placeholder = n_tiles.size() > 1;
      if (dma) {
        src << "  static constexpr int BM = " << dm << ", BN = " << (placeholder ? "ACCY_N_TILE" : std::to_string(dn))
            << ", STAGES = 4;\n};\n";
      } else {
        src << "  static constexpr int BM = " << BM << ", BN = " << BN << ", BK = " << BK << ", WAVES_M = " << WM
            << ", WAVES_N = " << WN << ";\n};\n";
      }
      int threads = dma ? 256 : WM * WN * 64;
      src << "extern \"C\" __global__ void __launch_bounds__(" << threads << ") " << nm << "(" << w->params() << ") {\n"
          << "  accy::gemm::" << (dma ? "mma16_dma" : "mma16") << "<Cfg_" << nm << ">(" << a << " + " << gs.a.offset
          << "L, " << b << " + " << gs.b.offset << "L, Epi_" << nm << "{" << inits.str() << "});\n}\n";
      k.source = src.str();
      if (placeholder) {
        k.tuning_key = tuning_key("gemm", k.source, "m=" + std::to_string(gs.m) + ",n=" + std::to_string(gs.n) +
                                                        ",k=" + std::to_string(gs.k) + ",batch=" + std::to_string(gs.batch));
        k.candidate_count = (uint32_t)n_tiles.size();
        k.candidate = candidate_for(k.tuning_key, k.candidate_count);
        dn = n_tiles[k.candidate];
        const std::string mark = "ACCY_N_TILE";
        k.source.replace(k.source.find(mark), mark.size(), std::to_string(dn));
      }
      int64_t tiles = dma ? ((gs.m + dm - 1) / dm) * ((gs.n + dn - 1) / dn) : ((gs.m + BM - 1) / BM) * ((gs.n + BN - 1) / BN);
      k.grid[0] = (uint32_t)tiles;
      k.block[0] = threads;
      k.shared_bytes = dma ? 0u : 2u * (BM + BN) * (BK + 8) * 2u;
    }
    if (k.source.empty()) k.source = src.str();
    k.name = nm;
    k.grid[1] = (uint32_t)gs.batch;
    k.klass = "gemm";
    k.label = "gemm:%" + std::to_string(v) + (target != v ? "+%" + std::to_string(target) : "");
    k.algorithmic_flops = 2.0 * (double)gs.batch * (double)gs.m * (double)gs.n * (double)gs.k;
    push(std::move(k), *w);
    if (target != v) {
      done_[v] = true;
      finish(target);
    } else {
      finish(v);
    }
  }

  // ---- sum over k of mul(A, B): the same contraction, spelled elementwise ----
  //
  // reduce_sum_K(mul(broadcast_in_dim(A), broadcast_in_dim(B))) where every reduced axis comes from
  // both A and B is dot_general(A, B) with those axes contracted, the kept axes of both as batch
  // axes and the rest free. runCpu rounds each product to the element type before summing; the
  // matrix cores form exact products (a difference inside the contraction tolerances), so this is
  // used only where the MFMA kernels apply.
  struct Operand {
    uint32_t src = 0;
    std::vector<int> to_mul;  // per source dim: the mul dim it becomes
  };

  bool operand_of(uint32_t u, size_t rank, Operand& o) const {
    const Op& op = g_.ops[u];
    if (op.kind == Kind::broadcast_in_dim) {
      o.src = op.args[0];
      o.to_mul.assign(op.ints.begin(), op.ints.end());
    } else {
      if (op.result.rank() != rank) return false;
      o.src = u;
      o.to_mul.resize(rank);
      for (size_t i = 0; i < rank; ++i) o.to_mul[i] = (int)i;
    }
    return true;
  }

  bool mulsum(uint32_t v) {
    const Op& red = g_.ops[v];
    if ((Reducer)red.code != Reducer::sum) return false;
    const DType d = red.result.dtype;
    if (d != DType::f32 && d != DType::bf16 && d != DType::f16) return false;
    double init;
    if (!splat_float(red.args[1], init) || init != 0.0) return false;
    const Op& mul = g_.ops[red.args[0]];
    if (mul.kind != Kind::binary || (Binary)mul.code != Binary::mul || mul.result.dtype != d) return false;
    const Type& mt = mul.result;
    const size_t R = mt.rank();
    Operand A, B;
    if (!operand_of(mul.args[0], R, A) || !operand_of(mul.args[1], R, B)) return false;
    // For each mul dim: the A / B source dim that supplies it (-1 if broadcast there).
    std::vector<int> from_a(R, -1), from_b(R, -1);
    const Type& at = g_.type(A.src);
    const Type& bt = g_.type(B.src);
    for (size_t i = 0; i < A.to_mul.size(); ++i)
      if (at.dims[i].extent == mt.dims[(size_t)A.to_mul[i]].extent && at.dims[i].extent != 1) from_a[(size_t)A.to_mul[i]] = (int)i;
    for (size_t i = 0; i < B.to_mul.size(); ++i)
      if (bt.dims[i].extent == mt.dims[(size_t)B.to_mul[i]].extent && bt.dims[i].extent != 1) from_b[(size_t)B.to_mul[i]] = (int)i;
    std::vector<bool> reduced(R, false);
    for (int64_t a : red.ints) reduced[(size_t)a] = true;
    Op dot;
    dot.kind = Kind::dot_general;
    dot.args = {A.src, B.src};
    std::vector<Dim> batch_dims, lf_dims, rf_dims;
    std::vector<size_t> batch_mul, lf_mul, rf_mul;
    for (size_t i = 0; i < R; ++i) {
      if (mt.dims[i].extent == 1) {
        // Size-one axes: must not come from a real axis of both (nothing to contract or batch).
        continue;
      }
      const bool ia = from_a[i] >= 0, ib = from_b[i] >= 0;
      if (reduced[i]) {
        if (!ia || !ib) return false;
        dot.lhs_contract.push_back(from_a[i]);
        dot.rhs_contract.push_back(from_b[i]);
      } else if (ia && ib) {
        dot.lhs_batch.push_back(from_a[i]);
        dot.rhs_batch.push_back(from_b[i]);
        batch_dims.push_back(mt.dims[i]);
        batch_mul.push_back(i);
      } else if (ia) {
        lf_dims.push_back(mt.dims[i]);
        lf_mul.push_back(i);
      } else if (ib) {
        rf_dims.push_back(mt.dims[i]);
        rf_mul.push_back(i);
      } else {
        return false;
      }
    }
    // Source dims that are not used (size one, or broadcast away) must have extent one.
    auto covered = [](const std::vector<int>& from, size_t src_dim) {
      return std::find(from.begin(), from.end(), (int)src_dim) != from.end();
    };
    for (size_t i = 0; i < at.rank(); ++i)
      if (!covered(from_a, i) && at.dims[i].extent != 1) return false;
    for (size_t i = 0; i < bt.rank(); ++i)
      if (!covered(from_b, i) && bt.dims[i].extent != 1) return false;
    // The contraction's free dims must flatten in the order the sources hold them; the dot result
    // is [batch, lhs free, rhs free].
    dot.result.dtype = d;
    for (auto* g : {&batch_dims, &lf_dims, &rf_dims})
      for (const Dim& x : *g) dot.result.dims.push_back(x);
    if (dot.lhs_contract.empty()) return false;
    GemmShape gs;
    if (!gemm_eligible(dot, gs)) return false;
    // Matrix cores only pay when both output extents fill a tile; x * x summed over an axis (a
    // norm) stays a row reduction.
    if (gs.m < 32 || gs.n < 32) return false;
    // Output strides: the reduce result keeps the non-reduced mul dims in order.
    std::vector<int64_t> rstr = row_major_strides(red.result.dims);
    std::vector<int> res_pos(R, -1);
    for (size_t i = 0, r = 0; i < R; ++i)
      if (!reduced[i]) res_pos[i] = (int)r++;
    auto group = [&](const std::vector<size_t>& muls, int64_t& extent, int64_t& stride) {
      std::vector<Dim> dims;
      std::vector<int64_t> strides;
      std::vector<size_t> idx;
      for (size_t j = 0; j < muls.size(); ++j) {
        dims.push_back(mt.dims[muls[j]]);
        strides.push_back(rstr[(size_t)res_pos[muls[j]]]);
        idx.push_back(j);
      }
      return flatten(dims, strides, idx, extent, stride);
    };
    OutStrides os;
    int64_t e;
    if (!group(batch_mul, e, os.b) || !group(lf_mul, e, os.m) || !group(rf_mul, e, os.n)) return false;
    gemm(v, gs, os);
    return true;
  }

  // ---- dot_general with runCpu's per-output serial k order ----
  void dot_serial(uint32_t v) {
    const Op& op = g_.ops[v];
    const Type& L = g_.type(op.args[0]);
    const Type& R = g_.type(op.args[1]);
    const Type& rt = op.result;
    int out = slots_.slot_of[v] >= 0 ? slots_.slot_of[v] : temp_slot(v);
    uint64_t nout = rt.elements();
    if (nout == 0) {
      finish(v);
      return;
    }
    auto in = [](const std::vector<int64_t>& a, size_t d) { return std::find(a.begin(), a.end(), (int64_t)d) != a.end(); };
    std::vector<Dim> cdims;
    for (int64_t a : op.lhs_contract) cdims.push_back(L.dims[(size_t)a]);
    uint64_t kn = prod(cdims, 0, cdims.size());
    DType d = rt.dtype;
    KernelWriter w(g_, slots_, itype());
    std::ostringstream body;
    std::vector<std::string> oc = delinearize("o", rt.dims);
    size_t nb = op.lhs_batch.size();
    size_t nlf = 0;
    for (size_t i = 0; i < L.rank(); ++i)
      if (!in(op.lhs_contract, i) && !in(op.lhs_batch, i)) ++nlf;
    std::string at = is_int(d) ? unsigned_type(d) : compute_type(d);
    body << "    " << at << " acc = (" << at << ")0;\n";
    body << "    for (I k = 0; k < (I)" << kn << "; ++k) {\n";
    Scope sc(body, "      ");
    std::vector<std::string> kc = delinearize("k", cdims);
    std::vector<std::string> lc(L.rank()), rc(R.rank());
    size_t f = 0;
    for (size_t i = 0; i < L.rank(); ++i) {
      auto b = std::find(op.lhs_batch.begin(), op.lhs_batch.end(), (int64_t)i);
      auto c = std::find(op.lhs_contract.begin(), op.lhs_contract.end(), (int64_t)i);
      if (b != op.lhs_batch.end()) lc[i] = oc[(size_t)(b - op.lhs_batch.begin())];
      else if (c != op.lhs_contract.end()) lc[i] = kc[(size_t)(c - op.lhs_contract.begin())];
      else lc[i] = oc[nb + f++];
    }
    f = 0;
    for (size_t i = 0; i < R.rank(); ++i) {
      auto b = std::find(op.rhs_batch.begin(), op.rhs_batch.end(), (int64_t)i);
      auto c = std::find(op.rhs_contract.begin(), op.rhs_contract.end(), (int64_t)i);
      if (b != op.rhs_batch.end()) rc[i] = oc[(size_t)(b - op.rhs_batch.begin())];
      else if (c != op.rhs_contract.end()) rc[i] = kc[(size_t)(c - op.rhs_contract.begin())];
      else rc[i] = oc[nb + nlf + f++];
    }
    std::string a = w.value(op.args[0], lc, sc);
    std::string b = w.value(op.args[1], rc, sc);
    if (is_int(d)) {
      body << "      acc = acc + (" << at << ")" << a << " * (" << at << ")" << b << ";\n";
    } else {
      body << "      const " << at << " prod = " << a << " * " << b << ";\n      acc = acc + prod;\n";
    }
    body << "    }\n";
    std::string res = is_int(d) ? "(" + std::string(compute_type(d)) + ")acc" : round_to(d, "acc");
    body << "    " << w.store(out, "o", d, res) << "\n";
    const uint32_t B = 256;
    std::string nm = name("dot", v);
    std::ostringstream src;
    src << "extern \"C\" __global__ void __launch_bounds__(" << B << ") " << nm << "(" << w.params() << ") {\n"
        << "  typedef " << w.itype << " I;\n"
        << "  for (I o = (I)blockIdx.x * " << B << " + threadIdx.x; o < (I)" << nout << "; o += (I)gridDim.x * "
        << B << ") {\n"
        << body.str() << "  }\n}\n";
    KernelStep k;
    k.source = src.str();
    k.name = nm;
    k.grid[0] = grid_for(nout, B, 65536);
    k.block[0] = B;
    k.klass = "dot";
    k.label = "dot:%" + std::to_string(v);
    k.algorithmic_flops = 2.0 * (double)nout * (double)kn;
    push(std::move(k), w);
    finish(v);
  }

  // ---- scatter_add: copy the input, then add updates in order, one (pre, post) position per thread ----
  void scatter_add(uint32_t v) {
    const Op& op = g_.ops[v];
    const Type& rt = op.result;
    int out = slots_.slot_of[v] >= 0 ? slots_.slot_of[v] : temp_slot(v);
    map_into(op.args[0], out);
    const Type& it = g_.type(op.args[1]);
    size_t axis = (size_t)op.axis;
    uint64_t pre = prod(rt.dims, 0, axis), post = prod(rt.dims, axis + 1, rt.rank());
    uint64_t ni = it.elements();
    int64_t ext = rt.dims[axis].extent;
    uint64_t work = pre * post;
    if (work == 0 || ni == 0) {
      finish(v);
      return;
    }
    DType d = rt.dtype;
    KernelWriter w(g_, slots_, itype());
    std::ostringstream body;
    body << "    const I p = w / (I)" << post << ", q = w % (I)" << post << ";\n";
    body << "    for (I j = 0; j < (I)" << ni << "; ++j) {\n";
    Scope sc(body, "      ");
    std::vector<std::string> jc = delinearize("j", it.dims);
    std::string idx = w.value(op.args[1], jc, sc);
    std::vector<Dim> udims = g_.type(op.args[2]).dims;
    std::vector<std::string> pc = delinearize("p", std::vector<Dim>(rt.dims.begin(), rt.dims.begin() + axis));
    std::vector<std::string> qc =
        delinearize("q", std::vector<Dim>(rt.dims.begin() + axis + 1, rt.dims.end()));
    std::vector<std::string> uc = pc;
    uc.insert(uc.end(), jc.begin(), jc.end());
    uc.insert(uc.end(), qc.begin(), qc.end());
    std::string u = w.value(op.args[2], uc, sc);
    body << "      const I kk = (I)(" << idx << " < 0 ? 0 : (" << idx << " > " << ext - 1 << " ? " << ext - 1 << " : "
         << idx << "));\n";
    body << "      const I dst = (p * (I)" << ext << " + kk) * (I)" << post << " + q;\n";
    std::string cur = w.load(out, "dst", d);
    std::string sum;
    if (is_float_domain(d) || d == DType::f64) sum = round_to(d, "(" + cur + " + " + u + ")");
    else sum = "accy::wadd<" + std::string(compute_type(d)) + "," + unsigned_type(d) + ">(" + cur + ", " + u + ")";
    body << "      " << w.store(out, "dst", d, sum) << "\n    }\n";
    // The output is read and written: drop the const qualifier on its parameter.
    w.arg(out, true);
    const uint32_t B = 256;
    std::string nm = name("scatter", v);
    std::ostringstream src;
    std::string params = w.params();
    src << "extern \"C\" __global__ void __launch_bounds__(" << B << ") " << nm << "(" << params << ") {\n"
        << "  typedef " << w.itype << " I;\n"
        << "  for (I w = (I)blockIdx.x * " << B << " + threadIdx.x; w < (I)" << work << "; w += (I)gridDim.x * " << B
        << ") {\n"
        << body.str() << "  }\n}\n";
    KernelStep k;
    k.source = src.str();
    k.name = nm;
    k.grid[0] = grid_for(work, B, 65536);
    k.block[0] = B;
    k.klass = "scatter";
    k.label = "scatter:%" + std::to_string(v);
    push(std::move(k), w);
    finish(v);
  }
};

// Lowest finite value of a float dtype as its storage bytes (`lowerFloatLowestConstant`,
// src/tensor/lower.zig:1005-1029): f16 -65504, bf16 the truncated -floatMax(f32), f32 / f64 -floatMax.
std::string lowest_finite_bytes(DType dt) {
  std::string b(dtype_size(dt), '\0');
  switch (dt) {
    case DType::f16: { const uint16_t h = 0xFBFF; std::memcpy(&b[0], &h, 2); break; }
    case DType::bf16: { const uint16_t h = f32_to_bf16_trunc(-3.40282347e+38f); std::memcpy(&b[0], &h, 2); break; }
    case DType::f32: { const float f = -3.40282347e+38f; std::memcpy(&b[0], &f, 4); break; }
    case DType::f64: { const double d = -1.7976931348623157e+308; std::memcpy(&b[0], &d, 8); break; }
    default: fail(Err::Unsupported, "sparse_cross_entropy on a non-float dtype");
  }
  return b;
}

// sparse_cross_entropy in the expanded form runCpu lowers it to (no kernel library;
// `lowerSparseCrossEntropyExpanded`, src/tensor/lower.zig:914-1003), with m the row max from the
// lowest finite value, over the class axis:
//   loss = log(sum(exp(x - m))) - sum(select(iota == target, x - m, 0)).
// The planner then fuses the three row reductions like any other (one row kernel per loss).
Graph expand_sparse_cross_entropy(const Graph& g) {
  Graph out;
  out.name = g.name;
  std::vector<uint32_t> id(g.ops.size());
  auto push = [&](Op op) {
    out.ops.push_back(std::move(op));
    return (uint32_t)(out.ops.size() - 1);
  };
  for (size_t i = 0; i < g.ops.size(); ++i) {
    const Op& src = g.ops[i];
    if (src.kind != Kind::sparse_cross_entropy) {
      Op op = src;
      for (uint32_t& a : op.args) a = id[a];
      id[i] = push(std::move(op));
      continue;
    }
    const uint32_t x = id[src.args[0]], t = id[src.args[1]];
    const Type lt = out.ops[x].result;  // a copy: push() below grows out.ops
    const int64_t axis = src.axis;
    std::vector<int64_t> keep;  // positions of the non-class axes
    for (int64_t d = 0; d < (int64_t)lt.rank(); ++d)
      if (d != axis) keep.push_back(d);
    const Type scalar{lt.dtype, {}}, row = src.result, idx{DType::i32, lt.dims}, mask{DType::i1, lt.dims};
    auto constant = [&](std::string bytes) {
      Op c; c.kind = Kind::constant; c.result = scalar; c.bytes = std::move(bytes);
      return push(std::move(c));
    };
    auto reduce = [&](uint32_t a, uint32_t init, Reducer r) {
      Op o; o.kind = Kind::reduce; o.code = (uint8_t)r; o.result = row; o.args = {a, init}; o.ints = {axis};
      return push(std::move(o));
    };
    auto expand = [&](uint32_t a, const Type& to, std::vector<int64_t> dims) {
      Op o; o.kind = Kind::broadcast_in_dim; o.result = to; o.args = {a}; o.ints = std::move(dims);
      return push(std::move(o));
    };
    auto elementwise = [&](Kind k, uint8_t code, const Type& to, std::vector<uint32_t> args) {
      Op o; o.kind = k; o.code = code; o.result = to; o.args = std::move(args);
      return push(std::move(o));
    };
    const uint32_t lowest = constant(lowest_finite_bytes(lt.dtype));
    const uint32_t zero = constant(std::string(dtype_size(lt.dtype), '\0'));
    const uint32_t m = reduce(x, lowest, Reducer::max);
    const uint32_t shifted = elementwise(Kind::binary, (uint8_t)Binary::sub, lt, {x, expand(m, lt, keep)});
    const uint32_t e = elementwise(Kind::unary, (uint8_t)Unary::exp, lt, {shifted});
    const uint32_t log_denominator = elementwise(Kind::unary, (uint8_t)Unary::log, row, {reduce(e, zero, Reducer::sum)});
    Op io; io.kind = Kind::iota; io.result = idx; io.axis = axis;
    const uint32_t positions = push(std::move(io));
    const uint32_t hit = elementwise(Kind::compare, (uint8_t)Cmp::eq, mask, {positions, expand(t, idx, keep)});
    const uint32_t selected = elementwise(Kind::select, 0, lt, {hit, shifted, expand(zero, lt, {})});
    const uint32_t picked = reduce(selected, zero, Reducer::sum);
    id[i] = elementwise(Kind::binary, (uint8_t)Binary::sub, row, {log_denominator, picked});
  }
  for (uint32_t p : g.params) out.params.push_back(id[p]);
  for (uint32_t o : g.outputs) out.outputs.push_back(id[o]);
  return out;
}

}  // namespace

Plan lower(const Program& program, const LowerOptions& options) {
  for (const Op& op : program.ops)
    if (op.kind == Kind::sparse_cross_entropy) {
      const Graph expanded = expand_sparse_cross_entropy(program);
      return Planner(expanded, options).run();
    }
  return Planner(program, options).run();
}

}  // namespace accy
