// Kernel formation, shared by the planner's translation units: the Planner class (one per lowered
// program) and the helpers its parts use. planner.cpp holds the walk over the program, scans, maps,
// launch tuning, serial contractions and scatter_add; planner_reduce.cpp the folds and row kernels;
// planner_views.cpp strided views and materialised transposes; planner_contraction.cpp the matrix-core
// contractions, grouped launches and epilogues; planner_attention.cpp the fused attention matcher and
// kernels. The fusion rules and their references are described in lower.cpp.
#pragma once

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
namespace planning {
using namespace detail;

inline bool is_inlinable(Kind k) {
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
inline std::optional<std::string> quad_base(const std::string& off) {
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

inline uint64_t prod(const std::vector<Dim>& dims, size_t b, size_t e) {
  uint64_t n = 1;
  for (size_t i = b; i < e; ++i) n *= (uint64_t)dims[i].extent;
  return n;
}

// 32-bit indices while every element index plus one grid stride (at most 2^20 workgroups x 256
// threads = 2^28) stays below 2^31, so that no grid-stride loop's increment overflows.
inline std::string index_type(uint64_t max_elems) { return max_elems < (1ull << 31) - (1ull << 28) ? "i32_t" : "i64_t"; }

inline uint32_t grid_for(uint64_t work_items, uint32_t block, uint64_t cap = 1u << 20) {
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
inline std::string transpose_tile(const std::string& et, int64_t R, int64_t C, int64_t sc, int64_t ds, const std::string& src,
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
inline int transpose_lanes(size_t elem_bytes, const std::vector<int64_t>& multiples) {
  for (int e : {std::max<int>(4, (int)(16 / elem_bytes)), 4}) {
    bool ok = true;
    for (int64_t x : multiples) ok = ok && x % e == 0;
    if (ok) return e;
  }
  return 1;
}

inline const char* reducer_op(Reducer r) {
  switch (r) {
    case Reducer::sum: return "accy::SumOp()";
    case Reducer::max: return "accy::MaxOp()";
    case Reducer::min: return "accy::MinOp()";
  }
  return "";
}

// Accumulator type of a reduction: f32 for 16-bit floats (reduction.zig:847, 861 widen f16), the
// unsigned twin for integer sums so wrap-around is defined.
inline std::string acc_type(DType d, Reducer r) {
  if (is_int(d) && r == Reducer::sum) return unsigned_type(d);
  return compute_type(d);
}

// The step of a serial fold (fold and chunked fold kernels): as fold_step, with float max / min that
// keep the later element on ties, as runCpu's fold does (accy::fold_max / fold_min).
inline std::string serial_fold_step(DType d, Reducer r, const std::string& acc, const std::string& x);

inline std::string fold_step(DType d, Reducer r, const std::string& acc, const std::string& x) {
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

inline std::string serial_fold_step(DType d, Reducer r, const std::string& acc, const std::string& x) {
  if ((is_float_domain(d) || d == DType::f64) && r != Reducer::sum)
    return std::string(r == Reducer::max ? "accy::fold_max(" : "accy::fold_min(") + acc + ", " + x + ")";
  return fold_step(d, r, acc, x);
}

class Planner {
 public:
  Planner(const Graph& g, const LowerOptions& o) : g_(g), opt_(o), slots_(g, plan_) {
    for (const Op& op : g.ops) max_elems_ = std::max<uint64_t>(max_elems_, op.result.elements());
  }

  Plan run();

 private:
  const Graph& g_;
  LowerOptions opt_;
  Plan plan_;
  Slots slots_;
  std::vector<bool> live_, needed_, done_;
  std::vector<std::vector<uint32_t>> users_;  // live operations reading each value (top-level graph)
  std::vector<bool> is_output_;
  int counter_ = 0;
  uint64_t max_elems_ = 1;

  // Index arithmetic is 32-bit unless some value of the program has 2^31 or more elements.
  std::string itype() const { return index_type(max_elems_); }

  void process(uint32_t v);

  void mark_live();
  // True when some reader of v other than the operations in `inside` (one kernel's values) can need
  // v from memory: an output, or a reader that is not elementwise, reached directly or through
  // elementwise operations (which other kernels would evaluate again from their operands).
  bool read_outside(uint32_t v, const std::set<uint32_t>& inside) const;

  int temp_slot(uint32_t v);

  std::string name(const char* klass, uint32_t v);

  void push(KernelStep k, const KernelWriter& w);

  void finish(uint32_t v);

  // Slot of value a, materialised by a map kernel when so far it is only evaluated inline.
  int materialize(uint32_t a);

  // ---- scan: the body's own plan, run as a host loop over two sets of carry buffers ----
  // The scan's value is carry 0 and projection i is carry i (builder.zig:899-990); a carry without a
  // reader gets no result slot.
  void scan(uint32_t v);

  // ---- map: out[i] = value at i ----
  void map(uint32_t v);

  void map_into(uint32_t v, int slot);

  // ---- fold: one output per thread, serial left-to-right over the reduced index ----
  void fold(uint32_t v);

  // The value a chunk's fold starts from, so that folding the chunks' partials in order from the
  // program's init gives the serial fold's result: -0 for a float sum (x + -0 = x for every x,
  // including -0), NaN for a float max / min (fold_max / fold_min skip a NaN second operand and return
  // the second operand when the first is NaN, so NaN is the absent element; ties keep the later
  // element, which the in-order combination of the chunks preserves), 0 for a
  // wrapping integer sum, the type's extreme for an integer max / min. Integer folds and float max /
  // min are then bit-identical to the serial fold; a float sum is associated differently (within the
  // reductions' 1e-5 relative bound). Empty for other dtypes.
  static std::optional<std::string> chunk_identity(DType d, Reducer r);

  // Partial dtype of a chunked fold: f32 for the 16-bit floats and f32, f64, the unsigned type for a
  // wrapping integer sum, the dtype itself for an integer max / min.
  static DType partial_dtype(DType d, Reducer r);

  // Kernel 1: output o, chunk s (blockIdx.y) folds reduced indices [s * chunk, (s + 1) * chunk) in
  // order from the chunk identity into part[s * nout + o]. Kernel 2: each output folds its S partials
  // in chunk order from the program's init, then rounds once (16-bit dtypes) and stores.
  void fold_chunked(uint32_t v, int out, const Type& in, const std::vector<size_t>& red, const std::vector<size_t>& keep,
                    const std::vector<Dim>& rdims, const std::vector<Dim>& kdims, uint64_t nout, uint64_t nred, Reducer r,
                    DType d);

  // ---- row group: fused reductions over trailing axes of one row space, one workgroup per row ----
  struct RowShape {
    std::vector<Dim> K, T;
  };

  bool row_shape(uint32_t v, RowShape& rs) const;

  struct RowKernel {
    std::vector<uint32_t> reduces, row_vals, full_vals;
  };

  bool row_group(uint32_t r0);

  std::vector<int> last_args_;

  void push_row(KernelStep k);

  bool try_row(const RowShape& rs, const RowKernel& rk);

  KernelStep gen_row(const RowShape& rs, const RowKernel& rk, bool commit);

  std::map<std::string, std::set<int>> probe_use_;

  // ---- launch tuning ----
  size_t kernel_index() const;
  // Key of a tunable kernel: device family, class, fingerprint of its default source and a readable
  // shape.
  static std::string tuning_key(const std::string& klass, const std::string& source, const std::string& shape);
  // Candidate for the next kernel step: forced (measurement), else the table's selection, else 0.
  uint32_t candidate_for(const std::string& key, uint32_t count) const;

  // ---- strided views: a value that is a transpose / rename / broadcast of a buffer ----
  struct View {
    int slot = -1;
    int64_t offset = 0;
    std::vector<int64_t> strides;  // per dim of the viewed value, in elements
  };

  bool resolve_view(uint32_t v, View& out) const;

  // A value that is a permutation of a buffer (a transpose view) whose innermost axis is strided in
  // the source while another axis r is contiguous there: a copy through LDS, one 64 x 64 tile of
  // (r, innermost) per workgroup, read along r and written along the innermost axis, so both sides
  // touch whole lines (an element-wise map would read one line per element). The other axes are
  // enumerated by blockIdx.y. Raw storage is copied, so any dtype.
  bool permute_copy(uint32_t v, int slot, const View& pv);

  // Collapses a group of dims (in the given order) into one extent and stride, if the group is
  // contiguous in the view; an empty group is extent 1, stride 0.
  static bool flatten(const std::vector<Dim>& dims, const std::vector<int64_t>& strides,
                      const std::vector<size_t>& group, int64_t& extent, int64_t& stride);

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

  bool gemm_shape(const Op& op, GemmShape& gs) const;

  // Direct-to-LDS tile sizes for the 16-bit kernel (0: not applicable).
  static int dma_rows(int64_t extent);

  // Operand layouts the direct-to-LDS kernel can stage: K-contiguous (the innermost contraction run
  // has stride 1 and whole 32-wide k tiles) or row-contiguous (the innermost row run has stride 1
  // and whole row tiles); every other stride and the offset 16-byte aligned.
  static bool dma_operand(const Group& rows, const Group& k, const Group& batch, int64_t offset, int tile, bool& kc);

  bool dma_eligible(const GemmShape& gs, int& dm, int& dn, bool& a_kc, bool& b_kc) const;

  // The f32 MFMA kernel's operand layouts: A K-contiguous, B N-contiguous, rows 16-byte aligned.
  static bool f32_layout_ok(const GemmShape& gs);

  // Copies an f32 operand view (batch x R x C with strides sb, sr, sc from offset `off` of `slot`) into
  // a new contiguous temporary [batch][R][C] and returns its slot. One workgroup per 64 x 64 tile: when
  // the rows are the contiguous axis (sr == 1, a transpose) the tile goes through LDS, read along r and
  // written along c, so both sides touch whole lines; otherwise element by element along c.
  int pack_f32(int slot, int64_t off, int64_t batch, int64_t R, int64_t C, int64_t sb, int64_t sr, int64_t sc);

  // Repacks the operands of a large f32 contraction whose layout the MFMA kernel does not take.
  void pack_f32_operands(GemmShape& gs);

  // The MFMA templates take 16-bit operands whose K or M/N stride is 1, with 8-element aligned rows
  // (or, for operands whose groups span several axes, the direct-to-LDS kernel's layouts).
  bool gemm_eligible(const Op& op, GemmShape& gs) const;

  // Marks dot operands that are not plain views of a buffer: they are materialised first (by the
  // kernel that produces them, e.g. as a full-row output of a row kernel).
  void mark_gemm_operands();

  // True when `v` is a (transpose / rename / broadcast) view of a parameter or an anchor value.
  bool view_chain_to_anchor(uint32_t v) const;

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
  bool splat_float(uint32_t v, double& out) const;

  // `v` = broadcast_in_dim(src) of a rank R-1 value back over the last axis of rank R.
  bool row_broadcast_of(uint32_t v, size_t R, uint32_t& src) const;

  bool reduces_last(const Op& op, size_t R) const;

  // Which axis of its own type the integer value `v` equals the coordinate of (iota seen through
  // broadcast_in_dim), or -1.
  int index_axis(uint32_t v) const;

  // `pred` (rank R) is true exactly where key index <= query index (query axis R-2, key axis R-1).
  bool causal_mask(uint32_t pred, size_t R) const;

  bool match_attention(uint32_t pv, Attn& at) const;

  void match_attentions();

  struct AttnLayout {
    int64_t sq = 0, sk = 0, nb = 1, q_s = 0, k_s = 0, v_s = 0, hd = 0;
    std::vector<int64_t> extents, q_b, k_b, v_b;  // batch axes: extents and per-operand strides
    View q, k, v;
  };

  static int free_axis(size_t rank, const std::vector<int64_t>& batch, const std::vector<int64_t>& contract);

  bool attention_layout(uint32_t pv, const Attn& at, AttnLayout& L) const;

  // Element offset of flattened (row-major) batch index b for one operand.
  static std::string batch_offset(const std::vector<int64_t>& extents, const std::vector<int64_t>& strides,
                                  int64_t offset);

  void attention(uint32_t pv, const Attn& at, const AttnLayout& L);

  // Score pairs the kernel computes: all of them, or those with key <= query under the causal mask.
  static double attention_pairs(const Attn& at, const AttnLayout& L);

  // f32 attention of head dimension 64 (attn::flash_f32): 32 queries per wave.
  void attention_f32(uint32_t pv, const Attn& at, const AttnLayout& L);


  void dot(uint32_t v);

  // ---- grouped contractions: several contractions of one activation in one launch ----
  //
  // dot_general v and the later, not yet planned contractions u with the same A view (same buffer,
  // offset and layout), the same extents and the same B layout, whose B operands are already
  // available and whose results are plain stores (no fused epilogue, no attention): the projections
  // of one normalised activation. They run as one direct-to-LDS launch of G x tiles workgroups
  // (mma16_dma_group), so the machine fills and drains once instead of G times. Every output keeps
  // its own k order and accumulation, so the results are those of separate launches bit for bit.
  static bool same_group(const Group& x, const Group& y);

  bool plain_store(uint32_t u) const;

  bool gemm_siblings(uint32_t v, const GemmShape& gs, std::vector<std::pair<uint32_t, GemmShape>>& group) const;

  void gemm_group(const std::vector<std::pair<uint32_t, GemmShape>>& group);

  // Output layout of a contraction result: strides of the flattened batch, m and n groups.
  struct OutStrides {
    int64_t b = 0, m = 0, n = 1;
  };

  void gemm(uint32_t v, const GemmShape& gs);

  // ---- contraction epilogues ----
  //
  // When the contraction's value v is not itself materialised and every use of it runs through
  // elementwise operations of v's shape into exactly one materialised value u (an activation, a
  // residual add), the kernel's epilogue computes u from the accumulator and stores u: v never
  // travels through HBM. Other operands of u's expression are read at the same index.
  bool epilogue_target(uint32_t v, uint32_t& target) const;

  // A fused epilogue worth a lookup table: contraction and result both 16-bit, and the result a chain
  // of at least six elementwise operations whose leaves are the contraction value and splat float
  // constants only (no other tensor, no index), so it is a function of the rounded contraction value.
  bool lut_epilogue(uint32_t v, uint32_t target, DType d, DType td) const;

  // Writes the contraction described by gs into the slot of value v (laid out per os), or, with a
  // fused epilogue, the value that the elementwise region after v materialises.
  void gemm(uint32_t v, const GemmShape& gs, const OutStrides& os);

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

  bool operand_of(uint32_t u, size_t rank, Operand& o) const;

  bool mulsum(uint32_t v);

  // ---- dot_general with runCpu's per-output serial k order ----
  void dot_serial(uint32_t v);

  // ---- scatter_add: copy the input, then add updates in order, one (pre, post) position per thread ----
  void scatter_add(uint32_t v);
};

}  // namespace planning
}  // namespace accy
