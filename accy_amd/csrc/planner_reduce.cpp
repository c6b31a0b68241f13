// Kernel formation for reductions: serial folds (whole or in chunks) and row kernels (several fused
// reductions over the trailing axes of one row space, one workgroup per row).
#include "planner_internal.hpp"

namespace accy {
namespace planning {

// ---- fold: one output per thread, serial left-to-right over the reduced index ----

void Planner::fold(uint32_t v) {
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

std::optional<std::string> Planner::chunk_identity(DType d, Reducer r) {
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

DType Planner::partial_dtype(DType d, Reducer r) {
  if (is_float_domain(d)) return DType::f32;
  if (r == Reducer::sum && d == DType::i32) return DType::u32;
  if (r == Reducer::sum && d == DType::i64) return DType::u64;
  return d;
}

void Planner::fold_chunked(uint32_t v, int out, const Type& in, const std::vector<size_t>& red, const std::vector<size_t>& keep,
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

bool Planner::row_shape(uint32_t v, RowShape& rs) const {
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

bool Planner::row_group(uint32_t r0) {
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
  // A reduction whose value no other kernel reads stays in the kernel's registers (no slot, no
  // store): C2's row maximum and sum, a norm's sum of squares. (Storing them cost 4.7 µs of C2's
  // 163 µs in a standalone harness.)
  std::set<uint32_t> inside(rk.reduces.begin(), rk.reduces.end());
  inside.insert(rk.row_vals.begin(), rk.row_vals.end());
  inside.insert(rk.full_vals.begin(), rk.full_vals.end());
  for (uint32_t v : rk.reduces)
    if (is_output_[v] || read_outside(v, inside)) temp_slot(v);
  for (uint32_t v : rk.row_vals) temp_slot(v);
  for (uint32_t v : rk.full_vals) temp_slot(v);
  KernelStep k = gen_row(rs, rk, true);
  push_row(std::move(k));
  for (uint32_t v : rk.reduces) finish(v);
  for (uint32_t v : rk.row_vals) finish(v);
  for (uint32_t v : rk.full_vals) finish(v);
  return true;
}

void Planner::push_row(KernelStep k) {
  k.args = last_args_;
  double bytes = 0;
  for (int s : k.args) bytes += (double)plan_.slots[(size_t)s].bytes;
  k.algorithmic_bytes = bytes;
  Step st;
  st.type = Step::Kernel;
  st.kernel = std::move(k);
  plan_.steps.push_back(std::move(st));
}

bool Planner::try_row(const RowShape& rs, const RowKernel& rk) {
  try {
    gen_row(rs, rk, false);
    return true;
  } catch (const NotFusable&) {
    return false;
  }
}

KernelStep Planner::gen_row(const RowShape& rs, const RowKernel& rk, bool commit) {
  uint64_t tn = prod(rs.T, 0, rs.T.size()), kn = prod(rs.K, 0, rs.K.size());
  const uint32_t VEC = tn % 4 == 0 ? 4 : 1;
  uint64_t lanes = (tn + VEC - 1) / VEC;
  // Two waves per row: against one workgroup of four waves per row, C2's logsumexp went from 163-165 to
  // 159-161 µs and C1's tone from 58 to 56 µs on one box (four rounds), 162.0 -> 159.0 and 53.4 ->
  // 52.3 µs on another, and C2 161.5 -> 162.9 (C1 51.0 -> 50.2) on a third; 512 threads helped C2
  // alike but slowed C1 by 4 %, 1024 slowed C2 by 40 %. More workgroups per CU are in flight, each
  // meeting two waves at its barriers instead of four.
  uint32_t B = lanes >= 128 ? 128 : (uint32_t)std::max<uint64_t>(64, (lanes + 63) / 64 * 64);
  uint64_t E = (tn + (uint64_t)B * VEC - 1) / ((uint64_t)B * VEC);
  size_t passes = rk.reduces.size() + (rk.full_vals.empty() ? 0 : 1);
  // A row read by several passes is kept in registers when each thread holds at most 64 of its
  // elements; a row too long for that with 128 threads takes 256, 512 or 1024 threads if that makes it
  // fit (read once instead of once per pass; four waves per SIMD still have 128 registers each).
  if (passes >= 2 && E * VEC > 64) {
    for (uint32_t wide : {256u, 512u, 1024u}) {
      const uint64_t e = (tn + (uint64_t)wide * VEC - 1) / ((uint64_t)wide * VEC);
      if (e * VEC <= 64) {
        B = wide;
        E = e;
        break;
      }
    }
  }
  // Short rows, many of them: one wave per row and four rows per workgroup. The row's reductions then
  // stay inside the wave (no LDS exchange, no barrier), and a CU keeps up to 32 rows in flight instead
  // of one row per workgroup of four waves. (A C5 RMS norm: 8192 rows of 2048 bf16.)
  uint32_t R = 1;
  if (lanes <= 512 && kn >= 4 * 256) {
    R = 4;
    B = 64;
    E = (tn + (uint64_t)B * VEC - 1) / ((uint64_t)B * VEC);
  }
  const std::string tid = R > 1 ? "(I)(threadIdx.x & 63)" : "(I)threadIdx.x";
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
       << "      const I c0 = ((I)e * " << B << " + " << tid << ") * " << VEC << ";\n";
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
    // Every thread folds its share of the row, then the shares are combined. max / min may start
    // every share from the init (it is idempotent under them); a sum takes the init once, in the
    // first thread's share, and the others start from the additive identity (-0 for floats, so
    // that a share of -0 elements stays -0).
    if (r == Reducer::sum) {
      const std::string zero = is_int(d) ? "(" + at + ")0" : (d == DType::f64 ? "-0.0" : "-0.0f");
      body << "    " << at << " " << acc << " = " << tid << " == 0 ? (" << at << ")" << init << " : " << zero << ";\n";
    } else {
      body << "    " << at << " " << acc << " = (" << at << ")" << init << ";\n";
    }
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
    if (commit && slots_.slot_of[rk.reduces[j]] >= 0)
      body << "    if (" << tid << " == 0) " << w.store(slots_.slot_of[rk.reduces[j]], "row", d, red_var[j]) << "\n";
    avail = j + 1;
  }
  if (!rk.row_vals.empty()) {
    body << "    if (" << tid << " == 0) {\n";
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
  src << "extern \"C\" __global__ void __launch_bounds__(" << B * R << ") " << nm << "(" << w.params() << ") {\n"
      << "  typedef " << w.itype << " I;\n" << w.align_hints() << lds_decl;
  if (R > 1)
    src << "  for (I row = (I)blockIdx.x * " << R << " + (I)(threadIdx.x >> 6); row < (I)" << kn
        << "; row += (I)gridDim.x * " << R << ") {\n";
  else
    src << "  for (I row = blockIdx.x; row < (I)" << kn << "; row += gridDim.x) {\n";
  src << decls << body.str() << "  }\n}\n";
  k.source = src.str();
  k.grid[0] = (uint32_t)std::min<uint64_t>((kn + R - 1) / R, 1u << 20);
  if (unroll_candidates.size() > 1) {
    k.tuning_key = tuning_key("row", k.source, "rows=" + std::to_string(kn) + ",cols=" + std::to_string(tn));
    k.candidate_count = (uint32_t)unroll_candidates.size();
    k.candidate = candidate_for(k.tuning_key, k.candidate_count);
    const std::string pragma = "#pragma unroll " + std::to_string(unroll_candidates[k.candidate]) + "\n";
    for (size_t at = k.source.find(kUnrollMark); at != std::string::npos; at = k.source.find(kUnrollMark, at))
      k.source.replace(at, std::strlen(kUnrollMark), pragma);
  }
  k.name = nm;
  k.block[0] = B * R;
  k.klass = "row";
  k.label = "row:%" + std::to_string(rk.reduces[0]);
  last_args_ = w.args;
  return k;
}

}  // namespace planning
}  // namespace accy
