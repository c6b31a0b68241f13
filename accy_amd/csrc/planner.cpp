// Kernel formation: walks the program in operation order and turns every value that must live in a
// device buffer into a generated kernel (the Planner's walk, scans, maps, launch tuning, serial
// contractions and scatter_add; the other parts are in planner_*.cpp). See lower.cpp for the fusion
// rules and the references.
#include "planner_internal.hpp"

namespace accy {
namespace planning {

Plan Planner::run() {
  size_t n = g_.ops.size();
  live_.assign(n, false);
  needed_.assign(n, false);
  done_.assign(n, false);
  mark_live();
  users_.assign(n, {});
  for (uint32_t v = 0; v < n; ++v)
    if (live_[v])
      for (uint32_t a : g_.ops[v].args) users_[a].push_back(v);
  is_output_.assign(n, false);
  for (uint32_t o : g_.outputs) is_output_[o] = true;
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

void Planner::process(uint32_t v) {
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

void Planner::mark_live() {
  std::vector<uint32_t> stack(g_.outputs.begin(), g_.outputs.end());
  while (!stack.empty()) {
    uint32_t v = stack.back();
    stack.pop_back();
    if (live_[v]) continue;
    live_[v] = true;
    for (uint32_t a : g_.ops[v].args) stack.push_back(a);
  }
}

bool Planner::read_outside(uint32_t v, const std::set<uint32_t>& inside) const {
  std::vector<uint32_t> stack = users_[v];
  std::set<uint32_t> seen;
  while (!stack.empty()) {
    const uint32_t u = stack.back();
    stack.pop_back();
    if (inside.count(u) || !seen.insert(u).second) continue;
    if (is_output_[u] || needed_[u] || !is_inlinable(g_.ops[u].kind)) return true;
    stack.insert(stack.end(), users_[u].begin(), users_[u].end());
  }
  return false;
}

int Planner::temp_slot(uint32_t v) {
  if (slots_.slot_of[v] < 0) {
    const Type& t = g_.type(v);
    slots_.slot_of[v] = slots_.add(SlotInfo::Temp, -1, t.dtype, t.bytes());
  }
  return slots_.slot_of[v];
}

std::string Planner::name(const char* klass, uint32_t v) {
  return std::string("accy_") + klass + "_" + std::to_string(counter_++) + "_v" + std::to_string(v);
}

void Planner::push(KernelStep k, const KernelWriter& w) {
  k.args = w.args;
  double bytes = 0;
  for (size_t i = 0; i < w.args.size(); ++i) bytes += (double)plan_.slots[(size_t)w.args[i]].bytes;
  k.algorithmic_bytes = bytes;
  Step st;
  st.type = Step::Kernel;
  st.kernel = std::move(k);
  plan_.steps.push_back(std::move(st));
}

void Planner::finish(uint32_t v) {
  done_[v] = true;
  slots_.produced[v] = true;
}

int Planner::materialize(uint32_t a) {
  int s = slots_.available(a);
  if (s >= 0) return s;
  if (!is_inlinable(g_.ops[a].kind)) fail(Err::Unsupported, "value not computed before its use");
  map(a);
  return slots_.available(a);
}

// ---- scan: the body's own plan, run as a host loop over two sets of carry buffers ----

void Planner::scan(uint32_t v) {
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

void Planner::map(uint32_t v) {
  map_into(v, slots_.slot_of[v] >= 0 ? slots_.slot_of[v] : temp_slot(v));
  finish(v);
}

void Planner::map_into(uint32_t v, int slot) {
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

// ---- launch tuning ----

size_t Planner::kernel_index() const {
  size_t n = 0;
  for (const Step& st : plan_.steps) n += st.type == Step::Kernel ? 1 : 0;
  return n;
}

std::string Planner::tuning_key(const std::string& klass, const std::string& source, const std::string& shape) {
  return "gfx950/" + klass + "/" + fingerprint(source) + "/" + shape;
}

uint32_t Planner::candidate_for(const std::string& key, uint32_t count) const {
  if (count <= 1) return 0;
  auto f = opt_.force_candidate.find(kernel_index());
  if (f != opt_.force_candidate.end()) return f->second < count ? f->second : 0;
  if (opt_.tuning)
    if (auto sel = opt_.tuning->find(key, count)) return sel->candidate;
  return 0;
}

// ---- dot_general with runCpu's per-output serial k order ----

void Planner::dot_serial(uint32_t v) {
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

void Planner::scatter_add(uint32_t v) {
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

}  // namespace planning

namespace {

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
      return planning::Planner(expanded, options).run();
    }
  return planning::Planner(program, options).run();
}

}  // namespace accy
