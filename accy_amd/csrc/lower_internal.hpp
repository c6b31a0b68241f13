// Internals shared by the planner (planner*.cpp) and the expression code generator (lower.cpp).
#pragma once

#include <functional>
#include <map>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "ir.hpp"
#include "plan.hpp"

namespace accy::detail {

// Raised while generating a fused kernel when a value cannot be computed inside it (a reduction of
// another row space, a result not produced yet). The planner then fuses less.
struct NotFusable : std::runtime_error {
  using std::runtime_error::runtime_error;
};

const char* compute_type(DType d);
const char* storage_type(DType d);
const char* unsigned_type(DType d);
bool is_float_domain(DType d);
bool is_int(DType d);
std::string round_to(DType d, const std::string& x);
std::string literal(DType d, const uint8_t* p);
std::string offset_expr(const std::vector<std::string>& coords, const std::vector<int64_t>& strides);
std::vector<std::string> delinearize(const std::string& lin, const std::vector<Dim>& dims);

// Device buffers of one plan and which values already live in them.
class Slots {
 public:
  Slots(const Graph& g, Plan& p);
  int add(SlotInfo::Role role, int io, DType d, uint64_t bytes);
  int available(uint32_t vid) const;  // slot of a value computed by an earlier step, or -1
  int constant(uint32_t vid);         // upload slot for a non-splat constant
  Plan& plan;
  std::vector<int> slot_of;
  std::vector<bool> produced;

 private:
  const Graph& g_;
  std::map<uint32_t, int> const_slot_;
};

// A block of generated statements with its own common-subexpression table.
struct Scope {
  std::ostringstream& out;
  std::string indent;
  std::map<std::string, std::string> memo;
  Scope(std::ostringstream& o, std::string ind) : out(o), indent(std::move(ind)) {}
};

// Builds the body of one generated kernel: collects the slots it touches (its parameters) and
// emits each value at a multi-index given as C expressions.
class KernelWriter {
 public:
  KernelWriter(const Graph& g, Slots& slots, const std::string& index_type);
  std::string value(uint32_t vid, const std::vector<std::string>& coords, Scope& sc);
  std::string arg(int slot, bool write);
  std::string load(int slot, const std::string& off, DType d);
  // Load of element `idx` past `base` (pointer-base form, so adjacent idx merge into vector loads).
  std::string load_at(int slot, const std::string& base, const std::string& idx, DType d);
  // Declaration of an aligned four-element load of slot at element offset base (an accy::Quad), and
  // element idx of such a variable converted to the compute type.
  std::string quad_load(int slot, const std::string& var, const std::string& base, DType d, bool stream = false);
  static std::string quad_elem(const std::string& var, const std::string& idx, DType d);
  std::string store(int slot, const std::string& off, DType d, const std::string& v);
  std::string tmp();
  std::string params() const;
  std::string align_hints() const;  // tells the compiler every buffer is 16-byte aligned

  // Lets a kernel supply values itself (a row kernel's own reduction results).
  std::function<bool(uint32_t, const std::vector<std::string>&, std::string&)> provide;
  // Lets a kernel serve a leaf load from registers (a row kernel's cached row).
  std::function<bool(int slot, const std::string& off, DType d, Scope& sc, std::string& out)> leaf_hook;

  std::vector<int> args;
  std::vector<bool> writes;
  std::string itype;

 private:
  const Graph& g_;
  Slots& slots_;
  int ntmp_ = 0;
};

}  // namespace accy::detail
