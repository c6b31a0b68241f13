// Kernel formation for strided views (transpose / rename / broadcast of a buffer) and materialised
// transposes through LDS tiles.
#include "planner_internal.hpp"

namespace accy {
namespace planning {

// ---- strided views: a value that is a transpose / rename / broadcast of a buffer ----

bool Planner::resolve_view(uint32_t v, View& out) const {
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

bool Planner::permute_copy(uint32_t v, int slot, const View& pv) {
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

bool Planner::flatten(const std::vector<Dim>& dims, const std::vector<int64_t>& strides,
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

}  // namespace planning
}  // namespace accy
