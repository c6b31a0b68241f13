// Kernel formation for fused attention: the matcher for dot(softmax_last(scale * dot(Q, K) [causal
// mask]), V) and the generated 16-bit and f32 flash kernels.
#include "planner_internal.hpp"

namespace accy {
namespace planning {

// ---- fused attention: dot(softmax_last(scale * dot(Q, K) [causal -inf mask]), V) ----

bool Planner::splat_float(uint32_t v, double& out) const {
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

bool Planner::row_broadcast_of(uint32_t v, size_t R, uint32_t& src) const {
  const Op& op = g_.ops[v];
  if (op.kind != Kind::broadcast_in_dim || op.ints.size() != R - 1 || op.result.rank() != R) return false;
  for (size_t i = 0; i + 1 < R; ++i)
    if (op.ints[i] != (int64_t)i) return false;
  src = op.args[0];
  return true;
}

bool Planner::reduces_last(const Op& op, size_t R) const {
  return op.kind == Kind::reduce && op.ints.size() == 1 && op.ints[0] == (int64_t)R - 1 &&
         g_.type(op.args[0]).rank() == R;
}

int Planner::index_axis(uint32_t v) const {
  const Op& op = g_.ops[v];
  if (op.kind == Kind::iota) return (int)op.axis;
  if (op.kind == Kind::broadcast_in_dim) {
    int a = index_axis(op.args[0]);
    return a < 0 ? -1 : (int)op.ints[(size_t)a];
  }
  return -1;
}

bool Planner::causal_mask(uint32_t pred, size_t R) const {
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

bool Planner::match_attention(uint32_t pv, Attn& at) const {
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

void Planner::match_attentions() {
  if (!opt_.allow_gemm) return;
  for (uint32_t v = 0; v < g_.ops.size(); ++v) {
    if (!live_[v] || g_.ops[v].kind != Kind::dot_general) continue;
    Attn at;
    if (!match_attention(v, at)) continue;
    for (uint32_t u : at.inner) done_[u] = true;
    attn_[v] = at;
  }
}

int Planner::free_axis(size_t rank, const std::vector<int64_t>& batch, const std::vector<int64_t>& contract) {
  int f = -1;
  for (size_t i = 0; i < rank; ++i) {
    if (std::find(batch.begin(), batch.end(), (int64_t)i) != batch.end()) continue;
    if (std::find(contract.begin(), contract.end(), (int64_t)i) != contract.end()) continue;
    if (f >= 0) return -2;
    f = (int)i;
  }
  return f;
}

bool Planner::attention_layout(uint32_t pv, const Attn& at, AttnLayout& L) const {
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
  // Head dimension (Q.K contraction and V's free axis, unit stride): 64 or 128 for 16-bit operands
  // (attn::flash), 64 for f32 (attn::flash_f32, the reference's flash pattern).
  const bool f32 = d.result.dtype == DType::f32;
  L.hd = qt.dims[qc].extent;
  if (f32 ? L.hd != 64 : (L.hd != 64 && L.hd != 128)) return false;
  if (kt.dims[kc].extent != L.hd || vt.dims[(size_t)vf].extent != L.hd) return false;
  if (L.q.strides[qc] != 1 || L.k.strides[kc] != 1 || L.v.strides[(size_t)vf] != 1) return false;
  L.sq = qt.dims[(size_t)qf].extent;
  L.sk = kt.dims[(size_t)kf].extent;
  // 32 queries per wave and key blocks of 32 (both kernels)
  if (vt.dims[vc].extent != L.sk || L.sq % 32 != 0 || L.sk % 32 != 0 || L.sq == 0 || L.sk == 0) return false;
  // Only shapes whose 16-bit kernel fits in 256 VGPRs without spilling fuse; the rest run unfused
  // (score contraction, softmax row kernel, P.V contraction). Head dimension 128 keeps Q^T, O^T and
  // two score tiles in 160 registers, which fits with multi-wave workgroups and one compiled loop
  // tail: it needs queries in blocks of 64 (a one-wave workgroup issues every K / V load itself and
  // keeps 16 load offsets), and under the causal mask query blocks and keys in multiples of 128, so
  // that every block's key-block count is 0 (mod 4). Head dimension 256 (Q^T, O^T and the scores
  // alone take 224 registers) always spilled. Spilling kernels are not only slow: the device
  // compiler has crashed compiling one (in its pass that rewrites MFMAs around AGPR spill copies),
  // taking the calling process with it. Head dimension 64 fits in every shape.
  if (!f32 && L.hd == 128) {
    if (L.sq % 64 != 0) return false;
    if (at.causal && (L.sq % 128 != 0 || L.sk % 128 != 0)) return false;
  }
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

std::string Planner::batch_offset(const std::vector<int64_t>& extents, const std::vector<int64_t>& strides,
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

void Planner::attention(uint32_t pv, const Attn& at, const AttnLayout& L) {
  const Op& d = g_.ops[pv];
  const DType dt = d.result.dtype;
  if (dt == DType::f32) {
    attention_f32(pv, at, L);
    return;
  }
  int out = slots_.slot_of[pv] >= 0 ? slots_.slot_of[pv] : temp_slot(pv);
  // Waves per workgroup (32 queries each): eight (two per SIMD) when the queries divide, else the
  // largest count that does, with two or more workgroups per CU; every wave's share of a K / V tile
  // (HD / 16 load instructions) must be whole.
  int waves = 1;
  for (int w : {8, 4, 2}) {
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
  // Two query blocks per workgroup (attn::blocks_per_group, the same rule): causal with an even
  // number of query blocks (complementary blocks, so every workgroup streams the same number of
  // keys), or unmasked when the pairs still fill whole rounds of 256 workgroups.
  const int64_t nqb = L.sq / (32 * waves);
  const int64_t pair = nqb % 2 == 0 && (at.causal || (L.nb * nqb) % 512 == 0) ? 2 : 1;
  ks.grid[0] = (uint32_t)(L.nb * nqb / pair);
  ks.block[0] = 64 * waves;  // one wave per 32 queries
  ks.klass = "attention";
  ks.label = "attention:%" + std::to_string(pv);
  ks.algorithmic_flops = 4.0 * (double)L.nb * attention_pairs(at, L) * (double)L.hd;
  push(std::move(ks), w);
  finish(pv);
}

double Planner::attention_pairs(const Attn& at, const AttnLayout& L) {
  double pairs = (double)L.sq * (double)L.sk;
  if (at.causal) {
    const double n = (double)std::min(L.sq, L.sk);
    pairs = n * (n + 1) / 2 + (L.sq > L.sk ? (double)(L.sq - L.sk) * (double)L.sk : 0.0);
  }
  return pairs;
}

void Planner::attention_f32(uint32_t pv, const Attn& at, const AttnLayout& L) {
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

}  // namespace planning
}  // namespace accy
