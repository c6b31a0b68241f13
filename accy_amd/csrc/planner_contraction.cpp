// Kernel formation for contractions on the matrix cores: operand layouts, f32 repacks, grouped
// launches of one activation's projections, fused epilogues (lookup tables included) and the
// elementwise mul + sum spelling.
#include <algorithm>

#include "planner_internal.hpp"

namespace accy {
namespace planning {

namespace {

// Tile-row group of the direct-to-LDS contraction's tile walk (gemm::GroupM): 4 when A is the larger
// operand (m > n), so that each XCD reads each of its A panels once per round where B is at least 8
// tiles wide and the operand read again is the smaller one; else 8. ACCY_GEMM_GROUP_M overrides the
// choice (1, 2, 4, 8 or 16). (Grouped launches keep 8: with their G contractions per tile, 4
// measured slower for the decoder's q, k and v projections, 204 against 201 µs.)
int tile_group_m(int64_t m, int64_t n) {
  if (const char* e = std::getenv("ACCY_GEMM_GROUP_M")) {
    const int g = std::atoi(e);
    if (g == 1 || g == 2 || g == 4 || g == 8 || g == 16) return g;
  }
  return m > n ? 4 : 8;
}

}  // namespace

// ---- strided views: a value that is a transpose / rename / broadcast of a buffer ----

bool Planner::gemm_shape(const Op& op, GemmShape& gs) const {
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

int Planner::dma_rows(int64_t extent) { return extent % 256 == 0 ? 256 : (extent % 128 == 0 ? 128 : 0); }

bool Planner::dma_operand(const Group& rows, const Group& k, const Group& batch, int64_t offset, int tile, bool& kc) {
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

bool Planner::dma_eligible(const GemmShape& gs, int& dm, int& dn, bool& a_kc, bool& b_kc) const {
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

bool Planner::f32_layout_ok(const GemmShape& gs) {
  auto ok4 = [](int64_t x) { return x % 4 == 0; };
  return gs.a_k == 1 && gs.b_n == 1 && ok4(gs.a_m) && ok4(gs.b_k) && ok4(gs.a_b) && ok4(gs.b_b) &&
         ok4(gs.a.offset) && ok4(gs.b.offset);
}

int Planner::pack_f32(int slot, int64_t off, int64_t batch, int64_t R, int64_t C, int64_t sb, int64_t sr, int64_t sc) {
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

void Planner::pack_f32_operands(GemmShape& gs) {
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

bool Planner::gemm_eligible(const Op& op, GemmShape& gs) const {
  if (!opt_.allow_gemm) return false;
  DType d = op.result.dtype;
  if (d != DType::bf16 && d != DType::f16 && d != DType::f32) return false;
  if (!gemm_shape(op, gs)) return false;
  if (gs.m == 0 || gs.n == 0 || gs.k == 0) return false;
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

void Planner::mark_gemm_operands() {
  for (uint32_t v = 0; v < g_.ops.size(); ++v) {
    const Op& op = g_.ops[v];
    if (!live_[v] || op.kind != Kind::dot_general || attn_.count(v)) continue;
    if (op.result.dtype != DType::bf16 && op.result.dtype != DType::f16 && op.result.dtype != DType::f32) continue;
    for (uint32_t a : op.args) {
      if (!view_chain_to_anchor(a)) needed_[a] = true;
    }
  }
}

bool Planner::view_chain_to_anchor(uint32_t v) const {
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

void Planner::dot(uint32_t v) {
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

bool Planner::same_group(const Group& x, const Group& y) { return x.ext == y.ext && x.str == y.str; }

bool Planner::plain_store(uint32_t u) const {
  uint32_t t;
  return attn_.find(u) == attn_.end() && !epilogue_target(u, t);
}

bool Planner::gemm_siblings(uint32_t v, const GemmShape& gs, std::vector<std::pair<uint32_t, GemmShape>>& group) const {
  const Op& op = g_.ops[v];
  const DType d = op.result.dtype;
  if (op.kind != Kind::dot_general || (d != DType::bf16 && d != DType::f16) || gs.multi) return false;
  // The decoder's three projections: 175.5 µs grouped against 186.6 µs in three launches (C5, one
  // box). ACCY_GEMM_NO_GROUP plans separate launches.
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

void Planner::gemm_group(const std::vector<std::pair<uint32_t, GemmShape>>& group) {
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
    cases << "      case " << i << ": return " << w.arg(out, true) << ";\n";
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
      << "  __device__ __forceinline__ u16_t* out(int g) const {\n"
      << "    switch (g) {\n" << cases.str() << "      default: return nullptr;\n    }\n  }\n"
      << "  __device__ __forceinline__ void operator()(u16_t* __restrict__ o, long b, long m, long n, float v) const {\n"
      << "    accy::" << (d == DType::bf16 ? "st_bf16" : "st_f16") << "(o, " << cidx << ", v);\n  }\n};\n";
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

void Planner::gemm(uint32_t v, const GemmShape& gs) {
  OutStrides os;
  os.b = gs.m * gs.n;
  os.m = gs.n;
  os.n = 1;
  gemm(v, gs, os);
}

// ---- contraction epilogues ----

bool Planner::epilogue_target(uint32_t v, uint32_t& target) const {
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

bool Planner::lut_epilogue(uint32_t v, uint32_t target, DType d, DType td) const {
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

void Planner::gemm(uint32_t v, const GemmShape& gs, const OutStrides& os) {
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
  // A 16-bit epilogue that reads buffers besides A, B and its output (a residual, a bias) goes
  // through LDS in whole row segments (gemm.h staged_epilogue; measured on C5's MLP-down: 224 ->
  // 219.7 us). A plain store does not (58.2 against 60.3 us staged for C5's q projection).
  const std::string ps = w->params();
  const long nparams = ps.empty() ? 0 : 1 + (long)std::count(ps.begin(), ps.end(), ',');
  const bool staged = table_members.empty() && target != v && (d == DType::bf16 || d == DType::f16) && nparams > 3 &&
                      !std::getenv("ACCY_GEMM_NO_STAGE");
  std::ostringstream src;
  KernelStep k;
  src << "#include \"gemm\"\n";
  src << "struct Epi_" << nm << " {\n" << members.str()
      << table_members << (staged ? "  static constexpr bool kStaged = true;\n" : "")
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
          << ", STAGES = 4, GROUP_M = " << tile_group_m(gs.m, gs.n) << ";\n};\n";
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

bool Planner::operand_of(uint32_t u, size_t rank, Operand& o) const {
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

bool Planner::mulsum(uint32_t v) {
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

}  // namespace planning
}  // namespace accy
