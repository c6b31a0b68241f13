// ACTP v1 codec. The decoder follows src/tensor/wire/decode.zig:31-120: frames for nested scan bodies,
// counts checked against the bytes left, ids checked against the values already defined in the
// frame, and every operation replayed through the checked Builder so no result type is taken from
// the bytes except where the layout carries it (parameter, constant, iota, custom_call types and the
// result dims of broadcast / broadcast_in_dim / reshape).
#include "wire.hpp"

#include <cstring>
#include <memory>

namespace accy::wire {
namespace {

struct Reader {
  const uint8_t* p;
  size_t len;
  size_t off = 0;
  size_t remaining() const { return len - off; }
  const uint8_t* take(size_t n) {
    if (n > remaining()) fail(Err::InvalidArtifact, "bytes end early");
    const uint8_t* r = p + off;
    off += n;
    return r;
  }
  uint32_t u32() {
    const uint8_t* b = take(4);
    return (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
  }
  int64_t i64() {
    const uint8_t* b = take(8);
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | b[i];
    return (int64_t)v;
  }
  std::string bytes() {
    uint32_t n = u32();
    const uint8_t* b = take(n);
    return std::string((const char*)b, n);
  }
};

struct ScanInfo {
  int64_t length = 0;
  std::vector<uint32_t> inits;
};

struct Frame {
  Builder builder;
  uint32_t remaining;
  ScanInfo scan;
  Frame(const std::string& name, uint32_t rem, ScanInfo s) : builder(name), remaining(rem), scan(std::move(s)) {}
};

template <typename E>
E decode_code(uint32_t v, int count) {
  if (v >= (uint32_t)count) fail(Err::UnknownTag);
  return (E)v;
}

class Decoder {
 public:
  Decoder(const uint8_t* b, size_t n) : r_{b, n} {}

  Program run() {
    if (r_.u32() != kMagic) fail(Err::BadMagic);
    if (r_.u32() != kVersion) fail(Err::UnsupportedVersion);
    std::string name = r_.bytes();
    open(name, {});
    // decode.zig:38-49 bounds the loop by the byte count; every step consumes at least one word.
    for (size_t step = 0; step <= r_.len; ++step) {
      Frame& f = *frames_.back();
      if (f.remaining != 0) {
        f.remaining -= 1;
        operation(f);
      } else if (frames_.size() == 1) {
        return finish(f);
      } else {
        close();
      }
    }
    fail(Err::InvalidArtifact);
  }

 private:
  Reader r_;
  std::vector<std::unique_ptr<Frame>> frames_;

  void open(const std::string& name, ScanInfo scan) {
    uint32_t remaining = r_.u32();
    frames_.push_back(std::make_unique<Frame>(name, remaining, std::move(scan)));
  }

  uint32_t count(size_t min_item_bytes) {
    uint32_t c = r_.u32();
    if (c > r_.remaining() / min_item_bytes) fail(Err::InvalidArtifact, "count past the end");
    return c;
  }

  uint32_t id(uint32_t limit) {
    uint32_t v = r_.u32();
    if (v >= limit) fail(Err::InvalidReference);
    return v;
  }

  std::vector<uint32_t> id_list(uint32_t limit, size_t max) {
    uint32_t c = count(4);
    if (c > max) fail(Err::TooManyOperands);
    std::vector<uint32_t> out(c);
    for (auto& v : out) v = id(limit);
    return out;
  }

  std::vector<int64_t> integers() {
    uint32_t c = count(8);
    std::vector<int64_t> out(c);
    for (auto& v : out) v = r_.i64();
    return out;
  }

  std::vector<Dim> dims() {
    uint32_t rank = count(4 + 8);
    std::vector<Dim> out(rank);
    for (auto& d : out) {
      d.name = r_.bytes();
      d.extent = r_.i64();
    }
    return out;
  }

  Type type() {
    DType dt = decode_code<DType>(r_.u32(), kDTypeCount);
    return Type{dt, dims()};
  }

  void operation(Frame& f) {
    Kind tag = decode_code<Kind>(r_.u32(), kKindCount);
    uint32_t limit = f.builder.size();
    Builder& b = f.builder;
    switch (tag) {
      case Kind::scan: {
        if (frames_.size() > kMaxScanDepth) fail(Err::ScanTooDeep);
        ScanInfo s;
        s.length = r_.i64();
        s.inits = id_list(limit, kMaxScanCarries);
        open("scan_body", std::move(s));
        return;
      }
      case Kind::parameter: b.input(type()); return;
      case Kind::constant: {
        Type t = type();
        std::string payload = r_.bytes();
        b.constant(t, payload);
        return;
      }
      case Kind::iota: {
        Type t = type();
        int64_t axis = r_.i64();
        b.iota(t, axis);
        return;
      }
      case Kind::custom_call: {
        Type t = type();
        std::string target = r_.bytes();
        uint32_t version = r_.u32();
        std::vector<uint32_t> operands = id_list(limit, kMaxCustomCallOperands);
        b.custom_call(target, version, operands, t);
        return;
      }
      case Kind::broadcast: {
        std::vector<Dim> d = dims();
        uint32_t in = id(limit);
        b.broadcast(in, d);
        return;
      }
      case Kind::broadcast_in_dim: {
        std::vector<Dim> d = dims();
        uint32_t in = id(limit);
        std::vector<int64_t> bd = integers();
        b.broadcast_in_dim(in, d, bd);
        return;
      }
      case Kind::reshape: {
        std::vector<Dim> d = dims();
        uint32_t in = id(limit);
        b.reshape(in, d);
        return;
      }
      case Kind::unary: {
        Unary u = decode_code<Unary>(r_.u32(), kUnaryCount);
        b.unary(u, id(limit));
        return;
      }
      case Kind::binary: {
        Binary op = decode_code<Binary>(r_.u32(), kBinaryCount);
        uint32_t l = id(limit), r = id(limit);
        b.binary(op, l, r);
        return;
      }
      case Kind::compare: {
        Cmp c = decode_code<Cmp>(r_.u32(), kCmpCount);
        uint32_t l = id(limit), r = id(limit);
        b.compare(c, l, r);
        return;
      }
      case Kind::select: {
        uint32_t p = id(limit), t = id(limit), e = id(limit);
        b.select(p, t, e);
        return;
      }
      case Kind::projection: {
        uint32_t src = id(limit);
        uint32_t index = r_.u32();
        b.projection(src, index);
        return;
      }
      case Kind::transpose: {
        uint32_t in = id(limit);
        b.transpose(in, integers());
        return;
      }
      case Kind::reduce: {
        uint32_t in = id(limit), init = id(limit);
        Reducer red = decode_code<Reducer>(r_.u32(), kReducerCount);
        b.reduce(in, init, red, integers());
        return;
      }
      case Kind::gather: {
        uint32_t in = id(limit), idx = id(limit);
        b.gather(in, idx, r_.i64());
        return;
      }
      case Kind::scatter_add: {
        uint32_t in = id(limit), idx = id(limit), upd = id(limit);
        b.scatter_add(in, idx, upd, r_.i64());
        return;
      }
      case Kind::sparse_cross_entropy: {
        uint32_t lg = id(limit), tg = id(limit);
        b.sparse_cross_entropy(lg, tg, r_.i64());
        return;
      }
      case Kind::dot_general: {
        uint32_t l = id(limit), r = id(limit);
        std::vector<int64_t> lc = integers(), rc = integers(), lb = integers(), rb = integers();
        b.dot_general(l, r, lc, rc, lb, rb);
        return;
      }
    }
    fail(Err::UnknownTag);
  }

  void close() {
    Frame& body = *frames_.back();
    uint32_t c = count(4);
    std::vector<uint32_t> outs(c);
    for (auto& o : outs) o = id(body.builder.size());
    auto graph = std::make_shared<Graph>(body.builder.finish(outs));
    ScanInfo scan = body.scan;
    frames_.pop_back();
    frames_.back()->builder.scan(scan.length, scan.inits, graph);
  }

  Program finish(Frame& root) {
    uint32_t c = count(4);
    std::vector<uint32_t> outs(c);
    for (auto& o : outs) o = id(root.builder.size());
    if (r_.off != r_.len) fail(Err::InvalidArtifact, "bytes after the program");
    return root.builder.finish(outs);
  }
};

struct Writer {
  std::vector<uint8_t> out;
  void u32(uint32_t v) {
    for (int i = 0; i < 4; ++i) out.push_back((uint8_t)(v >> (8 * i)));
  }
  void i64(int64_t v) {
    uint64_t u = (uint64_t)v;
    for (int i = 0; i < 8; ++i) out.push_back((uint8_t)(u >> (8 * i)));
  }
  void count(size_t n) {
    if (n > 0xffffffffull) fail(Err::InvalidArtifact, "list longer than a u32 count");
    u32((uint32_t)n);
  }
  void bytes(const std::string& s) {
    count(s.size());
    out.insert(out.end(), s.begin(), s.end());
  }
  void ids(const std::vector<uint32_t>& v) {
    for (uint32_t x : v) u32(x);
  }
  void id_list(const std::vector<uint32_t>& v) {
    count(v.size());
    ids(v);
  }
  void integers(const std::vector<int64_t>& v) {
    count(v.size());
    for (int64_t x : v) i64(x);
  }
  void dims(const std::vector<Dim>& d) {
    count(d.size());
    for (const Dim& x : d) {
      bytes(x.name);
      i64(x.extent);
    }
  }
  void type(const Type& t) {
    u32((uint32_t)t.dtype);
    dims(t.dims);
  }

  // Sink.graph (encode.zig:149-166): ids must be dense and parameters in parameter order.
  void graph_header(const Graph& g) {
    size_t pc = 0;
    for (size_t i = 0; i < g.ops.size(); ++i) {
      if (g.ops[i].kind != Kind::parameter) continue;
      if (g.ops[i].index != pc) fail(Err::InvalidProgram, "parameter out of order");
      if (pc == g.params.size()) fail(Err::InvalidProgram);
      if (g.params[pc] != i) fail(Err::InvalidProgram);
      ++pc;
    }
    if (pc != g.params.size()) fail(Err::InvalidProgram);
    count(g.ops.size());
  }

  void graph(const Graph& g, size_t depth) {
    graph_header(g);
    for (const Op& op : g.ops) {
      operation(op);
      if (op.kind == Kind::scan) {
        if (depth + 1 > kMaxScanDepth) fail(Err::ScanTooDeep);
        graph(*op.body, depth + 1);
      }
    }
    id_list(g.outputs);
  }

  void operation(const Op& op) {
    u32((uint32_t)op.kind);
    switch (op.kind) {
      case Kind::parameter: type(op.result); break;
      case Kind::constant: type(op.result); bytes(op.bytes); break;
      case Kind::iota: type(op.result); i64(op.axis); break;
      case Kind::custom_call:
        type(op.result);
        bytes(op.bytes);
        u32((uint32_t)op.index);
        id_list(op.args);
        break;
      case Kind::broadcast: dims(op.result.dims); u32(op.args[0]); break;
      case Kind::broadcast_in_dim: dims(op.result.dims); u32(op.args[0]); integers(op.ints); break;
      case Kind::reshape: dims(op.result.dims); u32(op.args[0]); break;
      case Kind::scan: i64(op.axis); id_list(op.args); break;
      case Kind::unary: u32(op.code); ids(op.args); break;
      case Kind::binary: u32(op.code); ids(op.args); break;
      case Kind::compare: u32(op.code); ids(op.args); break;
      case Kind::select: ids(op.args); break;
      case Kind::projection: u32(op.args[0]); count(op.index); break;
      case Kind::transpose: u32(op.args[0]); integers(op.ints); break;
      case Kind::reduce: ids(op.args); u32(op.code); integers(op.ints); break;
      case Kind::gather: ids(op.args); i64(op.axis); break;
      case Kind::scatter_add: ids(op.args); i64(op.axis); break;
      case Kind::sparse_cross_entropy: ids(op.args); i64(op.axis); break;
      case Kind::dot_general:
        ids(op.args);
        integers(op.lhs_contract);
        integers(op.rhs_contract);
        integers(op.lhs_batch);
        integers(op.rhs_batch);
        break;
    }
  }
};

}  // namespace

Program decode(const uint8_t* bytes, size_t len) {
  Decoder d(bytes, len);
  return d.run();
}

std::vector<uint8_t> encode(const Program& program) {
  Writer w;
  w.u32(kMagic);
  w.u32(kVersion);
  w.bytes(program.name);
  w.graph(program, 0);
  return std::move(w.out);
}

}  // namespace accy::wire
