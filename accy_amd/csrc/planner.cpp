// Kernel formation: walks the program in operation order and turns every value that must live in a
// device buffer into a generated kernel. See lower.cpp for the fusion rules and the references.
#include <algorithm>
#include <set>
#include <sstream>

#include "lower_internal.hpp"
#include "plan.hpp"

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

uint64_t prod(const std::vector<Dim>& dims, size_t b, size_t e) {
  uint64_t n = 1;
  for (size_t i = b; i < e; ++i) n *= (uint64_t)dims[i].extent;
  return n;
}

std::string index_type(uint64_t max_elems) { return max_elems < (1ull << 31) - 1 ? "i32_t" : "i64_t"; }

uint32_t grid_for(uint64_t work_items, uint32_t block, uint64_t cap = 1u << 20) {
  uint64_t g = (work_items + block - 1) / block;
  if (g == 0) g = 1;
  return (uint32_t)std::min<uint64_t>(g, cap);
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
    for (uint32_t v = 0; v < n; ++v) {
      if (!live_[v] || done_[v]) continue;
      const Op& op = g_.ops[v];
      switch (op.kind) {
        case Kind::parameter: break;
        case Kind::reduce:
          if (!row_group(v)) fold(v);
          break;
        case Kind::dot_general: dot_serial(v); break;
        case Kind::scatter_add: scatter_add(v); break;
        case Kind::scan: case Kind::projection: case Kind::custom_call: case Kind::sparse_cross_entropy:
          fail(Err::Unsupported, std::string(kind_name(op.kind)) + " is not supported by the HIP target");
        default:
          if (needed_[v]) map(v);
          break;
      }
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

  // ---- map: out[i] = value at i ----
  void map(uint32_t v) {
    map_into(v, slots_.slot_of[v] >= 0 ? slots_.slot_of[v] : temp_slot(v));
    finish(v);
  }

  void map_into(uint32_t v, int slot) {
    const Type& t = g_.type(v);
    uint64_t nel = t.elements();
    if (nel == 0) return;
    KernelWriter w(g_, slots_, itype());
    std::ostringstream body;
    Scope sc(body, "    ");
    std::vector<std::string> coords = delinearize("i", t.dims);
    std::string x = w.value(v, coords, sc);
    body << sc.indent << w.store(slot, "i", t.dtype, x) << "\n";
    const uint32_t B = 256;
    std::string nm = name("map", v);
    std::ostringstream src;
    src << "extern \"C\" __global__ void __launch_bounds__(" << B << ") " << nm << "(" << w.params() << ") {\n"
        << "  typedef " << w.itype << " I;\n"
        << "  for (I i = (I)blockIdx.x * " << B << " + threadIdx.x; i < (I)" << nel << "; i += (I)gridDim.x * " << B
        << ") {\n"
        << body.str() << "  }\n}\n";
    KernelStep k;
    k.source = src.str();
    k.name = nm;
    k.grid[0] = grid_for(nel, B, 65536);
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
    body << "      acc = " << fold_step(d, r, "acc", x) << ";\n    }\n";
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
    w.leaf_hook = [&](int slot, const std::string& off, DType d, Scope& sc, std::string& out) -> bool {
      bool varies = false;
      for (const auto& t : tc)
        if (t != "0" && off.find(t) != std::string::npos) varies = true;
      if (!varies) return false;
      std::string key = std::to_string(slot) + "|" + off;
      use_record[key].insert(cur_pass);
      auto it = leaf_array.find(key);
      if (it == leaf_array.end()) return false;
      std::string elem = it->second + "[e * " + std::to_string(VEC) + " + u]";
      if (leaf_first[key] == cur_pass) {
        sc.out << sc.indent << elem << " = " << w.load(slot, off, d) << ";\n";
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
    std::string loop_head;
    {
      std::ostringstream lh;
      lh << (unrolled ? "#pragma unroll\n" : "#pragma unroll 1\n") << "    for (int e = 0; e < " << E << "; ++e) {\n"
         << "#pragma unroll\n"
         << "      for (int u = 0; u < " << VEC << "; ++u) {\n"
         << "        const I c = ((I)e * " << B << " + (I)threadIdx.x) * " << VEC << " + u;\n";
      if (guard) lh << "        if (c < (I)" << tn << ") {\n";
      loop_head = lh.str();
    }
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
      body << loop_head;
      Scope inner(body, guard ? "          " : "        ");
      std::string x = w.value(op.args[0], full, inner);
      body << inner.indent << acc << " = " << fold_step(d, r, acc, x) << ";\n";
      body << loop_tail;
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
      body << loop_head;
      Scope sc(body, guard ? "          " : "        ");
      for (uint32_t v : rk.full_vals) {
        std::string x = w.value(v, full, sc);
        if (commit) body << sc.indent << w.store(slots_.slot_of[v], "row * (I)" + std::to_string(tn) + " + c", g_.type(v).dtype, x) << "\n";
      }
      body << loop_tail;
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
    k.name = nm;
    k.grid[0] = (uint32_t)std::min<uint64_t>(kn, 1u << 20);
    k.block[0] = B;
    k.klass = "row";
    k.label = "row:%" + std::to_string(rk.reduces[0]);
    last_args_ = w.args;
    return k;
  }

  std::map<std::string, std::set<int>> probe_use_;

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

}  // namespace

Plan lower(const Program& program, const LowerOptions& options) { return Planner(program, options).run(); }

}  // namespace accy
