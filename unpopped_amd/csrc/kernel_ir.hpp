// The kernel layer at the C-ABI boundary: a KernelFn as the JSON value tree serde writes for the
// reference's `KernelFn` (crates/unpopped/src/kernel.rs:1223-1250, with `ElementKind` as its
// variant name, crates/unpopped/src/text.rs:56-91, and a non-finite `Const` as a string tag,
// text.rs:241-276).  Enums are externally tagged: a unit variant is its name, any other variant
// is a one-key object {"Variant": payload}; a tuple variant's payload is an array, a struct
// variant's an object, a newtype's the inner value.
#pragma once

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace unp {
namespace kir {

struct J {
  enum Type { Null, Bool, Num, Str, Arr, Obj } t = Null;
  bool b = false;
  bool is_int = false;  // an integer literal, kept exactly in `i`
  int64_t i = 0;
  double d = 0.0;
  std::string s;
  std::vector<J> a;
  std::vector<std::pair<std::string, J>> o;

  static J null() { return J(); }
  static J boolean(bool v) {
    J j;
    j.t = Bool;
    j.b = v;
    return j;
  }
  static J integer(int64_t v) {
    J j;
    j.t = Num;
    j.is_int = true;
    j.i = v;
    j.d = (double)v;
    return j;
  }
  static J number(double v) {
    J j;
    j.t = Num;
    j.d = v;
    return j;
  }
  static J str(std::string v) {
    J j;
    j.t = Str;
    j.s = std::move(v);
    return j;
  }
  static J arr(std::vector<J> v = {}) {
    J j;
    j.t = Arr;
    j.a = std::move(v);
    return j;
  }
  static J obj(std::vector<std::pair<std::string, J>> v = {}) {
    J j;
    j.t = Obj;
    j.o = std::move(v);
    return j;
  }

  const J* get(const std::string& key) const;  // nullptr when absent or not an object
  bool operator==(const J& x) const;
  bool operator!=(const J& x) const { return !(*this == x); }
};

// Parse JSON text; on failure returns false and a message.
bool parse(const std::string& text, J& out, std::string& err);
// Compact JSON text.
std::string write(const J& j);

// ---- serde shapes ---------------------------------------------------------------------
inline J unit(const char* variant) { return J::str(variant); }
inline J var(const char* variant, J payload) { return J::obj({{variant, std::move(payload)}}); }
inline J tup(const char* variant, std::vector<J> items) { return var(variant, J::arr(std::move(items))); }

// ---- ScalarExpr (crates/unpopped/src/ir.rs:235-300) ------------------------------------
J e_const(double v);                        // Const(f64)
J e_int(int64_t v, const char* ek);         // ConstInt(i64, ElementKind)
J e_local(uint32_t l);                      // Local(u32)
J e_exec(const char* id, int axis = -1);    // Exec(ExecId): ThreadIdx(0) ... or a unit id
J e_add(J a, J b);
J e_sub(J a, J b);
J e_mul(J a, J b);
J e_div(J a, J b);
J e_bin(const char* op, J a, J b);          // Binary(BinaryOp, a, b)
J e_cast(J a, const char* to, const char* round = "NearestEven", const char* sat = "Wrap");
J e_bitcast(J a, const char* to);

// ---- Place / Stmt (crates/unpopped/src/kernel.rs:194-560) -------------------------------
J p_logical(uint32_t buffer, std::vector<J> coords);
J p_alloc(uint32_t alloc, J index);
J s_let(uint32_t local, J init);
J s_load(uint32_t local, J place);
J s_assign(uint32_t local, J value);
J s_store(J place, J value);
J s_if(J cond, std::vector<J> then, std::vector<J> els);
J s_for(uint32_t local, J start, J end, J step, std::vector<J> body);
J s_while(J cond, std::vector<J> body);
J s_barrier();  // Barrier { scope: Block, kind: Full } (kernel.rs:1177-1182)

// ---- KernelFn parts -------------------------------------------------------------------
J param_buffer(const std::string& name, const char* elem, const char* role, int rank /* -1: None */);
J param_scalar(const std::string& name, const char* ty, uint32_t local);
J local_decl(const char* elem);  // LocalDecl { elem, lanes: 1 }
J launch_shape(uint32_t block, uint32_t grid);  // LaunchShape::new([block,1,1],[grid,1,1])
J alloc_shared(const char* name, const char* elem, uint32_t extent);
J kernel_fn(const std::string& name, const char* compute, std::vector<J> params, std::vector<J> locals,
            std::vector<J> body, J launch, std::vector<J> allocs);

}  // namespace kir
}  // namespace unp
