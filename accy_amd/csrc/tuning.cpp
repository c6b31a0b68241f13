#include "tuning.hpp"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>

#include "ir.hpp"

namespace accy {

namespace {

void put_u32(std::vector<uint8_t>& o, uint32_t v) {
  for (int i = 0; i < 4; ++i) o.push_back((uint8_t)(v >> (8 * i)));
}
void put_u64(std::vector<uint8_t>& o, uint64_t v) {
  for (int i = 0; i < 8; ++i) o.push_back((uint8_t)(v >> (8 * i)));
}

struct Reader {
  const uint8_t* p;
  size_t n, at = 0;
  uint64_t uint(int bytes) {
    if (n - at < (size_t)bytes) fail(Err::InvalidArtifact, "tuning artifact truncated");
    uint64_t v = 0;
    for (int i = 0; i < bytes; ++i) v |= (uint64_t)p[at + i] << (8 * i);
    at += (size_t)bytes;
    return v;
  }
};

// A selection beats another when it is faster; equal times keep the one measured over more
// invocations, then the lower candidate (so merging is order-independent).
bool beats(const TuningSelection& a, const TuningSelection& b) {
  if (a.mean_ns != b.mean_ns) return a.mean_ns < b.mean_ns;
  if (a.samples != b.samples) return a.samples > b.samples;
  return a.candidate < b.candidate;
}

}  // namespace

std::optional<TuningSelection> TuningTable::find(const std::string& key, uint32_t candidate_count) const {
  std::lock_guard<std::mutex> lock(mu_);
  auto it = sel_.find({key, candidate_count});
  if (it == sel_.end()) return std::nullopt;
  return it->second;
}

void TuningTable::record(const std::string& key, uint32_t candidate_count, const TuningSelection& s) {
  if (key.empty() || s.candidate >= candidate_count || s.samples == 0)
    fail(Err::InvalidArtifact, "tuning record out of range");
  std::lock_guard<std::mutex> lock(mu_);
  auto [it, inserted] = sel_.emplace(std::make_pair(key, candidate_count), s);
  if (!inserted && beats(s, it->second)) it->second = s;
}

std::vector<uint8_t> TuningTable::encode() const {
  std::lock_guard<std::mutex> lock(mu_);
  std::vector<uint8_t> o;
  put_u32(o, kMagic);
  put_u32(o, kVersion);
  put_u32(o, (uint32_t)sel_.size());
  for (const auto& [k, s] : sel_) {
    put_u32(o, (uint32_t)k.first.size());
    o.insert(o.end(), k.first.begin(), k.first.end());
    put_u32(o, k.second);
    put_u32(o, s.candidate);
    put_u64(o, s.mean_ns);
    put_u32(o, s.samples);
  }
  return o;
}

void TuningTable::merge(const uint8_t* data, size_t len) {
  Reader r{data, len};
  if (r.uint(4) != kMagic) fail(Err::BadMagic, "not a tuning artifact");
  if (r.uint(4) != kVersion) fail(Err::UnsupportedVersion, "tuning artifact version");
  const uint64_t count = r.uint(4);
  std::vector<std::pair<std::pair<std::string, uint32_t>, TuningSelection>> recs;
  for (uint64_t i = 0; i < count; ++i) {
    const uint64_t kl = r.uint(4);
    if (kl == 0 || len - r.at < kl) fail(Err::InvalidArtifact, "tuning key length");
    std::string key((const char*)data + r.at, (size_t)kl);
    r.at += (size_t)kl;
    const uint32_t cc = (uint32_t)r.uint(4);
    TuningSelection s;
    s.candidate = (uint32_t)r.uint(4);
    s.mean_ns = r.uint(8);
    s.samples = (uint32_t)r.uint(4);
    if (s.candidate >= cc || s.samples == 0) fail(Err::InvalidArtifact, "tuning record out of range");
    recs.push_back({{std::move(key), cc}, s});
  }
  if (r.at != len) fail(Err::InvalidArtifact, "trailing bytes after tuning records");
  for (auto& [k, s] : recs) record(k.first, k.second, s);
}

size_t TuningTable::size() const {
  std::lock_guard<std::mutex> lock(mu_);
  return sel_.size();
}

void TuningTable::clear() {
  std::lock_guard<std::mutex> lock(mu_);
  sel_.clear();
}

TuningTable& process_tuning() {
  static TuningTable* table = [] {
    auto* t = new TuningTable();
    if (const char* path = std::getenv("ACCY_TUNING_FILE")) {
      std::ifstream f(path, std::ios::binary);
      if (f) {
        std::vector<uint8_t> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
        try {
          t->merge(bytes.data(), bytes.size());
        } catch (const Error& e) {
          std::fprintf(stderr, "accy: ignoring tuning file %s: %s\n", path, e.what());
        }
      }
    }
    return t;
  }();
  return *table;
}

std::string fingerprint(const std::string& s) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  char buf[17];
  std::snprintf(buf, sizeof buf, "%016llx", (unsigned long long)h);
  return buf;
}

}  // namespace accy
