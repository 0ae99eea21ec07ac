// The lifts the HIP backend lowers, restated in C++ over the serde JSON form of a KernelFn, and
// the recognizer behind Backend::lower_kernel.
//
// Each lift builds exactly the KernelFn the reference's lift builds (same statements, locals,
// parameters, launch shape and shared allocations), for the op forms this backend lowers:
// elementwise ops of n inputs (permuted reads included), reductions and scans of n inputs with a
// pre-map body and a fused post, the fused row folds, RowReduce, gathers with a body, and the int4
// dequant forms.  lower_kernel recognises a kernel by lifting
// every candidate form its signature admits and comparing the trees: a kernel equal to a lift's
// output is that form; anything else is refused with UnsupportedKernel (refuse rather than
// approximate, crates/unpopped/src/backend.rs:703-707).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <sstream>

#include "kernel_ir.hpp"
#include "unp_internal.hpp"

namespace unp {
namespace {

using kir::J;
using namespace kir;

// A LiftDecline (crates/unpopped/src/kernel_lift.rs:48-85): the variant and its reason.
struct Decline {
  std::string what;
};

const char* EK(int32_t kind) { return kind_name(kind); }
bool is_int_kernel_dtype(int32_t k) { return k == UNP_I32 || k == UNP_I64; }
bool pow2(uint32_t v) { return v != 0 && (v & (v - 1)) == 0; }

J thread() { return e_exec("ThreadIdx", 0); }
J as_i32(J e) { return e_cast(std::move(e), "I32"); }
J uconst(uint32_t v) { return e_int(v, "U32"); }
J int_(int64_t v) { return e_int(v, "I32"); }
J loc(uint32_t l) { return e_local(l); }

const char* reduce_op_name(int32_t op) {
  switch (op) {
    case UNP_OP_SUM: return "Sum";
    case UNP_OP_PROD: return "Prod";
    case UNP_OP_MAX: return "Max";
    case UNP_OP_MIN: return "Min";
    case UNP_OP_MEAN: return "Mean";
    case UNP_OP_AND: return "And";
    case UNP_OP_OR: return "Or";
    case UNP_OP_XOR: return "Xor";
    case UNP_OP_MAXNUM: return "MaxNum";
    case UNP_OP_MINNUM: return "MinNum";
    default: return nullptr;
  }
}
bool is_bit_op(int32_t op) { return op == UNP_OP_AND || op == UNP_OP_OR || op == UNP_OP_XOR; }
bool is_num_op(int32_t op) { return op == UNP_OP_MAXNUM || op == UNP_OP_MINNUM; }

// `for counter(d) in 0..extent(d) { inner }` (kernel_lift.rs:1037-1047).
std::vector<J> for_axis(uint32_t d, uint32_t r, std::vector<J> inner) {
  return {s_for(r + d, int_(0), loc(d), int_(1), std::move(inner))};
}

// The Max/Min/MaxNum/MinNum step (kernel_lift.rs:1097-1127): `if !have { acc = v }` else the NaN
// arm, then `have = 1`.  The NaN arm (nan_arm, :1129-1160): an integer just compares; Max/Min take
// a NaN element (`v != v`); MaxNum/MinNum replace a NaN accumulator (`acc != acc`) and compare only
// a non-NaN element (`v == v`).
std::vector<J> extremum_step(int32_t rop, uint32_t acc, uint32_t have, uint32_t val, bool is_int) {
  const char* better = (rop == UNP_OP_MAX || rop == UNP_OP_MAXNUM) ? "CmpGt" : "CmpLt";
  J keep_going = s_if(e_bin(better, loc(val), loc(acc)), {s_assign(acc, loc(val))}, {});
  J nan_check;
  if (is_int)
    nan_check = keep_going;
  else if (is_num_op(rop))
    nan_check = s_if(e_bin("CmpNe", loc(acc), loc(acc)), {s_assign(acc, loc(val))},
                     {s_if(e_bin("CmpEq", loc(val), loc(val)), {keep_going}, {})});
  else
    nan_check = s_if(e_bin("CmpNe", loc(val), loc(val)), {s_assign(acc, loc(val))}, {keep_going});
  return {s_if(loc(have), {nan_check}, {s_assign(acc, loc(val))}), s_assign(have, int_(1))};
}

// The And/Or/Xor step of an integer fold, seeded by the first element (bit_step,
// kernel_lift.rs:1071-1095): `if have { acc = acc OP v } else { acc = v }`, then `have = 1`.
std::vector<J> bit_step(int32_t rop, uint32_t acc, uint32_t have, uint32_t val) {
  const char* op = rop == UNP_OP_AND ? "BitAnd" : rop == UNP_OP_OR ? "BitOr" : "BitXor";
  return {s_if(loc(have), {s_assign(acc, e_bin(op, loc(acc), loc(val)))}, {s_assign(acc, loc(val))}),
          s_assign(have, int_(1))};
}

// The fold step (kernel_lift.rs:1049-1069).
std::vector<J> fold_step(int32_t rop, uint32_t acc, uint32_t have, uint32_t val, bool is_int) {
  switch (rop) {
    case UNP_OP_SUM:
    case UNP_OP_MEAN:
      return {s_assign(acc, e_add(loc(acc), loc(val)))};
    case UNP_OP_PROD:
      return {s_assign(acc, e_mul(loc(acc), loc(val)))};
    case UNP_OP_AND:
    case UNP_OP_OR:
    case UNP_OP_XOR:
      return bit_step(rop, acc, have, val);
    default:
      return extremum_step(rop, acc, have, val, is_int);
  }
}

// A float-to-float (or int-to-float) cast that rounds to nearest even (kernel_lift.rs:1027-1034).
J widen(J e, const char* to) { return e_cast(std::move(e), to); }

// ReductionShape (kernel_lift.rs:838-1025).
struct Shape {
  int32_t dtype;
  uint32_t r;
  uint32_t n = 1;
  std::vector<uint32_t> reduced, kept;
  uint32_t acc, have, val, red;

  Shape(int32_t dt, uint32_t rank, uint32_t axes_mask, uint32_t n_inputs = 1) : dtype(dt), r(rank), n(n_inputs) {
    if (axes_mask == 0) reduced.push_back(r - 1);
    else
      for (uint32_t d = 0; d < r; ++d)
        if (axes_mask & (1u << d)) reduced.push_back(d);
    for (uint32_t d = 0; d < r; ++d)
      if (std::find(reduced.begin(), reduced.end(), d) == reduced.end()) kept.push_back(d);
    acc = 2 * r + n;
    have = acc + 1;
    val = acc + 2;
    red = acc + 3;
  }
  uint32_t counter(uint32_t d) const { return r + d; }
  uint32_t loaded(uint32_t k) const { return 2 * r + k; }
  bool is_int() const { return is_int_kernel_dtype(dtype); }
  const char* acc_ty() const { return is_int() ? EK(dtype) : "F64"; }
  J up(J e) const { return (dtype == UNP_F64 || is_int()) ? e : widen(std::move(e), "F64"); }
  J fold_identity(int32_t rop) const {
    const bool one = rop == UNP_OP_PROD;
    return is_int() ? e_int(one ? 1 : 0, EK(dtype)) : up(e_const(one ? 1.0 : 0.0));
  }
  std::vector<J> counters() const {
    std::vector<J> c;
    for (uint32_t d = 0; d < r; ++d) c.push_back(loc(counter(d)));
    return c;
  }
  // reduce_loop (kernel_lift.rs:919-941): one load per input, `val = up(body)` with each
  // Input(k) bound to the k-th loaded local, the fold step, inside the reduced axes' loops.
  std::vector<J> reduce_loop(int32_t rop, const J& body) const {
    std::vector<J> inner;
    for (uint32_t k = 0; k < n; ++k) inner.push_back(s_load(loaded(k), p_logical(k, counters())));
    inner.push_back(s_let(val, up(subst_inputs(body))));
    for (auto& s : fold_step(rop, acc, have, val, is_int())) inner.push_back(s);
    for (auto it = reduced.rbegin(); it != reduced.rend(); ++it) inner = for_axis(*it, r, inner);
    return inner;
  }
  J subst_inputs(const J& body) const;
  // stored_value (kernel_lift.rs:987-1003): with a fused post, the fold rounded once into `red`
  // and the post over it.
  J stored_value(int32_t rop, const J* post, std::vector<J>& body) const;
  std::vector<J> out_coords(bool keepdim) const {
    std::vector<J> c;
    for (uint32_t d = 0; d < r; ++d) {
      const bool k = std::find(kept.begin(), kept.end(), d) != kept.end();
      if (k) c.push_back(loc(counter(d)));
      else if (keepdim) c.push_back(int_(0));
    }
    return c;
  }
  J stored(int32_t rop) const {
    J v = loc(acc);
    if (rop == UNP_OP_MEAN) {
      J div;
      bool first = true;
      for (uint32_t d : reduced) {
        J f = widen(loc(d), "F64");
        div = first ? f : e_mul(div, f);
        first = false;
      }
      v = e_div(v, div);
    }
    return (dtype == UNP_F64 || is_int()) ? v : widen(v, EK(dtype));
  }
  // signature (kernel_lift.rs:1006-1024).
  void signature(uint32_t out_rank, std::vector<J>& params, std::vector<J>& locals) const {
    params.clear();
    for (uint32_t k = 0; k < n; ++k) params.push_back(param_buffer("in" + std::to_string(k), EK(dtype), "Read", (int)r));
    params.push_back(param_buffer("out", EK(dtype), "Write", (int)out_rank));
    for (uint32_t d = 0; d < r; ++d) params.push_back(param_scalar("n" + std::to_string(d), "I32", d));
    locals.clear();
    for (uint32_t i = 0; i < 2 * r; ++i) locals.push_back(local_decl("I32"));
    for (uint32_t k = 0; k < n; ++k) locals.push_back(local_decl(EK(dtype)));
    locals.push_back(local_decl(acc_ty()));
    locals.push_back(local_decl("I32"));
    locals.push_back(local_decl(acc_ty()));
  }
};

// check_accumulated_dtype (kernel_lift.rs:763-803) for the ops lifted here: a bit or NaN-ignoring
// fold only in a plain reduction, a bit fold only at an integer dtype, and at an integer dtype no
// Mean and no fused post (`has_post`: the post is not the identity Reduced(0)).
void check_accumulated(int32_t dtype, int32_t rop, const char* what, bool has_post = false) {
  if (!reduce_op_name(rop)) throw Decline{"UnsupportedForm: a reduce op this restatement does not name"};
  if (((is_bit_op(rop) || is_num_op(rop)) && std::strcmp(what, "a reduction") != 0) ||
      (is_bit_op(rop) && !is_int_kernel_dtype(dtype)))
    throw Decline{"UnsupportedForm: a bit or NaN-ignoring reduction outside a plain reduction, or a bit reduction "
                  "at a float dtype"};
  if (dtype == UNP_F32 || dtype == UNP_F64) return;
  if (!is_int_kernel_dtype(dtype))
    throw Decline{std::string("UnsupportedForm: ") + what + " outside F32, F64, I32 and I64"};
  if (rop == UNP_OP_MEAN) throw Decline{"UnsupportedForm: an integer Mean"};
  if (has_post) throw Decline{"UnsupportedForm: a fused post at an integer dtype"};
}

void check_rank(int32_t rank) {
  if (rank < 1 || rank > 8) throw Decline{"BadRank"};
}

J launch_or_null(uint32_t block, uint32_t grid) { return (block || grid) ? launch_shape(block, grid) : J::null(); }

J input_leaf(uint32_t k);
J reduced_leaf(uint32_t t);
void check_reduction_exprs(const J& body, const J* post, uint32_t n_inputs);
void check_post(const J& e, int64_t available, int64_t n_inputs);
int64_t leaf_index(const J& e);
template <class F> J map_leaves(const J& e, const F& leaf);

// lift_reduction_opdef (kernel_lift.rs:447-484) and lift_reduction_opdef_launched
// (kernel_lift/block_reduce.rs:50-93): n inputs, a pre-map `body` over them (Input(0) for the
// plain fold) and an optional fused `post` over Reduced(0) (nullptr for the identity post).
J lift_reduction(const std::string& name, int32_t dtype, int32_t rank, int32_t rop, uint32_t axes, bool keepdim,
                 uint32_t block, uint32_t grid, uint32_t n_inputs = 1, const J* body_expr = nullptr,
                 const J* post = nullptr) {
  check_accumulated(dtype, rop, "a reduction", post && !(*post == reduced_leaf(0)));
  const J plain = input_leaf(0);
  const J& bexpr = body_expr ? *body_expr : plain;
  if (post && *post == reduced_leaf(0)) post = nullptr;  // the identity post
  check_reduction_exprs(bexpr, post, n_inputs);
  check_rank(rank);
  if (axes >> rank) throw Decline{"UnsupportedForm: a reduced axis outside the rank"};
  const Shape sh(dtype, (uint32_t)rank, axes, n_inputs);
  std::vector<J> params, locals;
  const uint32_t out_rank = keepdim ? sh.r : (uint32_t)sh.kept.size();
  sh.signature(out_rank, params, locals);
  if (!block && !grid) {
    std::vector<J> body = {s_let(sh.acc, sh.fold_identity(rop)), s_let(sh.have, int_(0))};
    for (auto& s : sh.reduce_loop(rop, bexpr)) body.push_back(s);
    const J value = sh.stored_value(rop, post, body);
    body.push_back(s_store(p_logical(sh.n, sh.out_coords(keepdim)), value));
    for (auto it = sh.kept.rbegin(); it != sh.kept.rend(); ++it) body = for_axis(*it, sh.r, body);
    if (post) locals.push_back(local_decl(EK(dtype)));  // red: the stage value rounded to the compute dtype
    return kernel_fn(name, EK(dtype), params, locals, body, J::null(), {});
  }
  if (grid == 0 || !pow2(block)) throw Decline{"BadLaunch"};
  // check_order_independent (block_reduce.rs:97-133)
  if (is_bit_op(rop) || is_num_op(rop))
    throw Decline{"UnsupportedForm: a bit or NaN-ignoring reduction in a launched reduction (the sequential lift "
                  "only)"};
  if ((rop == UNP_OP_PROD && !sh.is_int()) || (rop == UNP_OP_MEAN && sh.is_int()))
    throw Decline{"UnsupportedForm: an integer Mean or a float Prod in a launched reduction"};
  const bool flag = rop == UNP_OP_MAX || rop == UNP_OP_MIN;
  const uint32_t partner_have = sh.red + 1;
  auto publish = [&]() {
    std::vector<J> v = {s_store(p_alloc(0, as_i32(thread())), loc(sh.acc))};
    if (flag) v.push_back(s_store(p_alloc(1, as_i32(thread())), loc(sh.have)));
    return v;
  };
  std::vector<J> row = {s_let(sh.acc, sh.fold_identity(rop)), s_let(sh.have, int_(0))};
  std::vector<J> slice = sh.reduce_loop(rop, bexpr);
  // Tree::slice (block_reduce.rs:278-288): the outermost reduced loop starts at the thread
  // and steps by the block.
  J& f = slice[0].o[0].second;
  for (auto& kv : f.o) {
    if (kv.first == "start") kv.second = as_i32(thread());
    if (kv.first == "step") kv.second = as_i32(e_exec("BlockDim", 0));
  }
  for (auto& s : slice) row.push_back(s);
  for (auto& s : publish()) row.push_back(s);
  row.push_back(s_barrier());
  for (uint32_t s = block / 2; s > 0; s /= 2) {
    const J partner = as_i32(e_add(thread(), uconst(s)));
    std::vector<J> rb = {s_load(sh.val, p_alloc(0, partner))};
    const std::vector<J> combine = fold_step(rop, sh.acc, sh.have, sh.val, sh.is_int());
    if (flag) {
      rb.push_back(s_load(partner_have, p_alloc(1, partner)));
      rb.push_back(s_if(loc(partner_have), combine, {}));
    } else {
      for (auto& c : combine) rb.push_back(c);
    }
    for (auto& p : publish()) rb.push_back(p);
    row.push_back(s_if(e_bin("CmpLt", thread(), uconst(s)), rb, {}));
    row.push_back(s_barrier());
  }
  {
    // thread0_stores (block_reduce.rs:292-307)
    std::vector<J> then;
    const J value = sh.stored_value(rop, post, then);
    then.push_back(s_store(p_logical(sh.n, sh.out_coords(keepdim)), value));
    row.push_back(s_if(e_bin("CmpEq", thread(), uconst(0)), then, {}));
  }
  std::vector<J> body;
  if (sh.kept.empty()) {
    body = {s_if(e_bin("CmpEq", e_exec("BlockIdx", 0), uconst(0)), row, {})};
  } else {
    body = row;
    for (auto it = sh.kept.rbegin(); it != sh.kept.rend(); ++it) body = for_axis(*it, sh.r, body);
    J& outer = body[0].o[0].second;
    for (auto& kv : outer.o) {
      if (kv.first == "start") kv.second = as_i32(e_exec("BlockIdx", 0));
      if (kv.first == "step") kv.second = as_i32(e_exec("GridDim", 0));
    }
  }
  locals.push_back(local_decl(EK(dtype)));
  locals.push_back(local_decl("I32"));
  std::vector<J> allocs = {alloc_shared("partial", sh.acc_ty(), block)};
  if (flag) allocs.push_back(alloc_shared("partial_have", "I32", block));
  return kernel_fn(name, EK(dtype), params, locals, body, launch_shape(block, grid), allocs);
}

// scan_identity (kernel_lift.rs:712-753): the integer extremes, or the float identities with
// the infinities built by Bitcast of their bit patterns.
J scan_identity(int32_t rop, int32_t dtype) {
  if (is_int_kernel_dtype(dtype)) {
    const bool w = dtype == UNP_I64;
    const int64_t lo = w ? INT64_MIN : INT32_MIN, hi = w ? INT64_MAX : INT32_MAX;
    const int64_t v = rop == UNP_OP_PROD ? 1 : rop == UNP_OP_MAX ? lo : rop == UNP_OP_MIN ? hi : 0;
    return e_int(v, EK(dtype));
  }
  auto inf = [&](bool neg) {
    if (dtype == UNP_F64) {
      const uint64_t b = neg ? 0xFFF0000000000000ull : 0x7FF0000000000000ull;
      return e_bitcast(e_int((int64_t)b, "I64"), "F64");
    }
    const uint32_t b = neg ? 0xFF800000u : 0x7F800000u;
    return e_bitcast(e_int((int64_t)(int32_t)b, "I32"), EK(dtype));
  };
  switch (rop) {
    case UNP_OP_PROD: return e_const(1.0);
    case UNP_OP_MAX: return inf(true);
    case UNP_OP_MIN: return inf(false);
    default: return e_const(0.0);
  }
}

bool dtype_is_f64(const Shape& sh) { return sh.dtype == UNP_F64; }

// scan_loads (kernel_lift.rs:530-545): one load per input at the current position, then
// `val = up(pre)` with each Input(k) bound to the k-th loaded local.
std::vector<J> scan_loads(const Shape& sh, const J& pre) {
  std::vector<J> pass;
  for (uint32_t k = 0; k < sh.n; ++k) pass.push_back(s_load(sh.loaded(k), p_logical(k, sh.counters())));
  pass.push_back(s_let(sh.val, sh.up(sh.subst_inputs(pre))));
  return pass;
}

// scan_write (kernel_lift.rs:578-602): the prefix stored at the current position; with a fused
// post, the prefix rounded once into `red` and the post over it, its Input(k) leaves bound to
// the elements loaded for this position.
std::vector<J> scan_write(const Shape& sh, int32_t rop, const J* post) {
  // scan_stored (kernel_lift.rs:604-619): a running Mean divides by the count folded so far.
  J stored = sh.stored(rop);
  if (rop == UNP_OP_MEAN) {
    J mean = e_div(loc(sh.acc), widen(loc(sh.have), "F64"));
    stored = dtype_is_f64(sh) ? mean : widen(mean, EK(sh.dtype));
  }
  const J place = p_logical(sh.n, sh.counters());
  if (!post) return {s_store(place, stored)};
  const J value = map_leaves(*post, [&](const J& x, J& out) {
    if (x.t != J::Obj || x.o.size() != 1) return false;
    if (x.o[0].first == "Reduced") {
      out = loc(sh.red);
      return true;
    }
    if (x.o[0].first == "Input") {
      out = loc(sh.loaded((uint32_t)leaf_index(x)));
      return true;
    }
    return false;
  });
  return {s_let(sh.red, stored), s_store(place, value)};
}

// scan_pass (kernel_lift.rs:548-576): load and pre-map, fold, and write the prefix after the
// fold (inclusive) or before it (exclusive).
std::vector<J> scan_pass(const Shape& sh, int32_t rop, bool exclusive, const J& pre, const J* post) {
  std::vector<J> pass = scan_loads(sh, pre);
  const std::vector<J> write = scan_write(sh, rop, post);
  std::vector<J> fold = fold_step(rop, sh.acc, sh.have, sh.val, sh.is_int());
  if (rop == UNP_OP_MEAN) fold.push_back(s_assign(sh.have, e_add(loc(sh.have), int_(1))));
  if (exclusive) {
    for (auto& s : write) pass.push_back(s);
    for (auto& s : fold) pass.push_back(s);
  } else {
    for (auto& s : fold) pass.push_back(s);
    for (auto& s : write) pass.push_back(s);
  }
  return pass;
}

// check_scan (kernel_lift.rs:658-690) for the expressions: the pre-map reads only the op's
// inputs (leaves_ok); a fused post reads Reduced(0) and the inputs (check_post with one stage),
// and only at a float dtype (check_accumulated_dtype, kernel_lift.rs:796-801).
void check_scan_exprs(int32_t dtype, const J& pre, const J* post, uint32_t n_inputs) {
  check_post(pre, 0, (int64_t)n_inputs);
  if (post) {
    if (is_int_kernel_dtype(dtype)) throw Decline{"UnsupportedForm: a fused post at an integer dtype"};
    check_post(*post, 1, (int64_t)n_inputs);
  }
}

// lift_scan_opdef (kernel_lift.rs:504-519) and lift_scan_opdef_launched
// (kernel_lift/scan_launched.rs:54-102): n inputs, a pre-map `pre_expr` over them (Input(0) for
// the plain scan) and an optional fused `post` over Reduced(0) and the inputs (nullptr for the
// identity post).
J lift_scan(const std::string& name, int32_t dtype, int32_t rank, int32_t rop, int32_t axis, bool exclusive,
            bool reverse, uint32_t block, uint32_t grid, uint32_t n_inputs = 1, const J* pre_expr = nullptr,
            const J* post = nullptr) {
  check_accumulated(dtype, rop, "a scan", post && !(*post == reduced_leaf(0)));
  const J plain = input_leaf(0);
  const J& pre = pre_expr ? *pre_expr : plain;
  if (post && *post == reduced_leaf(0)) post = nullptr;  // the identity post
  check_scan_exprs(dtype, pre, post, n_inputs);
  check_rank(rank);
  const bool launched = block || grid;
  if (axis < 0 || axis >= rank) throw Decline{"UnsupportedForm: a scan axis outside the rank"};
  if (launched && axis != rank - 1) throw Decline{"UnsupportedForm: a scan over a non-innermost axis in a launched scan"};
  if (rop == UNP_OP_MEAN && dtype != UNP_F32 && dtype != UNP_F64) throw Decline{"UnsupportedForm: an integer Mean"};
  if (!launched) {
    const Shape sh(dtype, (uint32_t)rank, 1u << axis, n_inputs);
    const uint32_t scanned = sh.reduced[0];
    std::vector<J> pass = scan_pass(sh, rop, exclusive, pre, post);
    J start = reverse ? e_sub(loc(scanned), int_(1)) : int_(0);
    J end = reverse ? int_(-1) : loc(scanned);
    J step = reverse ? int_(-1) : int_(1);
    std::vector<J> row = {s_let(sh.acc, sh.up(scan_identity(rop, dtype))), s_let(sh.have, int_(0)),
                          s_for(sh.counter(scanned), start, end, step, pass)};
    for (auto it = sh.kept.rbegin(); it != sh.kept.rend(); ++it) row = for_axis(*it, sh.r, row);
    std::vector<J> params, locals;
    sh.signature(sh.r, params, locals);
    if (post) locals.push_back(local_decl(EK(dtype)));  // red: the prefix rounded to the compute dtype
    return kernel_fn(name, EK(dtype), params, locals, row, J::null(), {});
  }
  if (grid == 0 || !pow2(block)) throw Decline{"BadLaunch"};
  const Shape sh(dtype, (uint32_t)rank, 0, n_inputs);
  if (rop == UNP_OP_MEAN) throw Decline{"UnsupportedForm: a Mean scan in a launched scan"};
  if (rop == UNP_OP_PROD && !sh.is_int()) throw Decline{"UnsupportedForm: a float Prod scan in a launched scan"};
  const bool flag = rop == UNP_OP_MAX || rop == UNP_OP_MIN;
  const uint32_t base = sh.red + 1;
  const uint32_t chunk = base, lo = base + 1, hi = base + 2, partner = base + 3, flag_tmp = base + 4;
  const uint32_t scanned = sh.reduced[0];
  auto identity = [&]() { return sh.up(scan_identity(rop, dtype)); };
  auto tid = [&]() { return as_i32(thread()); };
  auto publish = [&]() {
    std::vector<J> v = {s_store(p_alloc(0, as_i32(thread())), loc(sh.acc))};
    if (flag) v.push_back(s_store(p_alloc(1, as_i32(thread())), loc(sh.have)));
    return v;
  };
  auto walk = [&](std::vector<J> body) {
    J n = loc(scanned);
    if (reverse)
      return s_for(sh.counter(scanned), e_sub(e_sub(n, int_(1)), loc(lo)), e_sub(e_sub(n, int_(1)), loc(hi)), int_(-1), body);
    return s_for(sh.counter(scanned), loc(lo), loc(hi), int_(1), body);
  };
  std::vector<J> fold_only = scan_loads(sh, pre);
  for (auto& s : fold_step(rop, sh.acc, sh.have, sh.val, sh.is_int())) fold_only.push_back(s);
  std::vector<J> row = {s_let(sh.acc, identity()), s_let(sh.have, int_(0)), s_let(partner, identity()), walk(fold_only)};
  for (auto& s : publish()) row.push_back(s);
  row.push_back(s_barrier());
  for (uint32_t d = 1; d < block; d *= 2) {
    J active = e_bin("CmpGe", thread(), uconst(d));
    std::vector<J> read = {s_load(sh.val, p_alloc(0, as_i32(e_sub(thread(), uconst(d))))), s_assign(partner, loc(sh.val))};
    std::vector<J> comb = fold_step(rop, sh.acc, sh.have, partner, sh.is_int());
    for (auto& s : publish()) comb.push_back(s);
    row.push_back(s_if(active, read, {}));
    row.push_back(s_barrier());
    row.push_back(s_if(active, comb, {}));
    row.push_back(s_barrier());
  }
  {
    const J prev = as_i32(e_sub(thread(), uconst(1)));
    std::vector<J> load = {s_load(sh.val, p_alloc(0, prev)), s_assign(sh.acc, loc(sh.val))};
    if (flag) {
      load.push_back(s_load(flag_tmp, p_alloc(1, prev)));
      load.push_back(s_assign(sh.have, loc(flag_tmp)));
    }
    row.push_back(s_if(e_bin("CmpEq", thread(), uconst(0)), {s_assign(sh.acc, identity()), s_assign(sh.have, int_(0))}, load));
  }
  row.push_back(walk(scan_pass(sh, rop, exclusive, pre, post)));
  row.push_back(s_barrier());
  std::vector<J> body;
  if (sh.kept.empty()) {
    body = {s_if(e_bin("CmpEq", e_exec("BlockIdx", 0), uconst(0)), row, {})};
  } else {
    body = row;
    for (auto it = sh.kept.rbegin(); it != sh.kept.rend(); ++it) body = for_axis(*it, sh.r, body);
    J& outer = body[0].o[0].second;
    for (auto& kv : outer.o) {
      if (kv.first == "start") kv.second = as_i32(e_exec("BlockIdx", 0));
      if (kv.first == "step") kv.second = as_i32(e_exec("GridDim", 0));
    }
  }
  // Scan::bounds (scan_launched.rs:173-207), spliced in front of the body.
  J n = loc(scanned);
  std::vector<J> bounds = {
      s_let(chunk, int_(0)),
      s_while(e_bin("CmpLt", e_mul(loc(chunk), int_(block)), n), {s_assign(chunk, e_add(loc(chunk), int_(1)))}),
      s_let(lo, e_mul(tid(), loc(chunk))),
      s_let(hi, e_bin("Min", e_add(loc(lo), loc(chunk)), n)),
  };
  body.insert(body.begin(), bounds.begin(), bounds.end());
  std::vector<J> params, locals;
  sh.signature(sh.r, params, locals);
  locals.push_back(local_decl(EK(dtype)));
  for (int i = 0; i < 3; ++i) locals.push_back(local_decl("I32"));
  locals.push_back(local_decl(sh.acc_ty()));
  locals.push_back(local_decl("I32"));
  std::vector<J> allocs = {alloc_shared("partial", sh.acc_ty(), block)};
  if (flag) allocs.push_back(alloc_shared("partial_have", "I32", block));
  return kernel_fn(name, EK(dtype), params, locals, body, launch_shape(block, grid), allocs);
}

// grid_stride_outermost (kernel_lift.rs:288-312): the outermost loop becomes a grid-stride loop.
void grid_stride(J& k, uint32_t block, uint32_t grid) {
  if (block == 0 || grid == 0) throw Decline{"BadLaunch"};
  J* body = nullptr;
  for (auto& kv : k.o)
    if (kv.first == "body") body = &kv.second;
  J& outer = body->a[0].o[0].second;
  for (auto& kv : outer.o) {
    if (kv.first == "start")
      kv.second = as_i32(e_add(e_mul(e_exec("BlockIdx", 0), e_exec("BlockDim", 0)), e_exec("ThreadIdx", 0)));
    if (kv.first == "step") kv.second = as_i32(e_mul(e_exec("GridDim", 0), e_exec("BlockDim", 0)));
  }
  for (auto& kv : k.o)
    if (kv.first == "launch") kv.second = launch_shape(block, grid);
}

void check_post(const J& e, int64_t available, int64_t n_inputs);
J input_leaf(uint32_t k);
int64_t leaf_index(const J& e);
template <class F> J map_leaves(const J& e, const F& leaf);

// lift_gather_opdef (kernel_lift/gather.rs:35-55, check_gather :64-101, cell :184-232): n inputs,
// input `index` the integer index (read at the output coordinate), input `data` the gathered one
// (read with its `axis` coordinate replaced by the clamped index), the others read at the output
// coordinate, and `body` an elementwise expression over Input(0..n) stored at the output
// coordinate (OpDef::gather is n = 2, data 0, index 1 and the identity body Input(0),
// ir.rs:3838-3855).  Launched by grid_stride.
J lift_gather(const std::string& name, int32_t dtype, int32_t rank, int32_t idx, int32_t axis, int32_t oob,
              uint32_t block, uint32_t grid, uint32_t n = 2, uint32_t data = 0, uint32_t index = 1,
              const J* body_expr = nullptr) {
  check_rank(rank);
  if (idx != UNP_I32 && idx != UNP_I64 && idx != UNP_U32) throw Decline{"UnsupportedForm: a non-integer gather index"};
  if (axis < 0 || axis >= rank || n < 2 || n > 8 || data >= n || index >= n || data == index)
    throw Decline{"UnsupportedForm: an ill-formed gather"};
  if (!kind_name(dtype) || kind_bytes(dtype) == 0) throw Decline{"UnsupportedForm: a gather of a sub-byte dtype"};
  const J plain = input_leaf(data);
  const J& bexpr = body_expr ? *body_expr : plain;
  check_post(bexpr, 0, (int64_t)n);  // leaves_ok: the inputs and constants only
  const uint32_t r = (uint32_t)rank;
  auto loaded = [&](uint32_t k) { return 2 * r + k; };
  const uint32_t extent = 2 * r + n, clamped = extent + 1;
  auto at = [&](uint32_t buffer, int via_axis, uint32_t via) {
    std::vector<J> c;
    for (uint32_t d = 0; d < r; ++d) c.push_back(((int)d == via_axis) ? loc(via) : loc(r + d));
    return p_logical(buffer, c);
  };
  auto ic = [&](int64_t v) { return e_int(v, EK(idx)); };
  J raw = loc(loaded(index));
  J clamp = e_bin("Min", e_bin("Max", raw, ic(0)), e_sub(loc(extent), ic(1)));
  J zero = (dtype == UNP_I32 || dtype == UNP_I64 || dtype == UNP_U32 || dtype == UNP_I8 || dtype == UNP_I16 ||
            dtype == UNP_U8 || dtype == UNP_U16 || dtype == UNP_U64)
               ? e_int(0, EK(dtype))
               : e_const(0.0);
  std::vector<J> compute;
  for (uint32_t k = 0; k < n; ++k)
    if (k != index) compute.push_back(s_load(loaded(k), k == data ? at(k, axis, clamped) : at(k, -1, 0)));
  const J value = map_leaves(bexpr, [&](const J& x, J& o) {
    if (x.t == J::Obj && x.o.size() == 1 && x.o[0].first == "Input") {
      o = loc(loaded((uint32_t)leaf_index(x)));
      return true;
    }
    return false;
  });
  compute.push_back(s_store(at(n, -1, 0), value));
  auto guarded = [&](std::vector<J> oobb) {
    J upper = s_if(e_bin("CmpGe", raw, loc(extent)), oobb, compute);
    return s_if(e_bin("CmpLt", raw, ic(0)), oobb, {upper});
  };
  std::vector<J> cell = {s_load(loaded(index), at(index, -1, 0)), s_let(clamped, clamp)};
  if (oob == UNP_OOB_SKIP) cell.push_back(guarded({}));
  else if (oob == UNP_OOB_ZEROFILL) cell.push_back(guarded({s_store(at(n, -1, 0), zero)}));
  else if (oob == UNP_OOB_CLAMP)
    for (auto& s : compute) cell.push_back(s);
  else throw Decline{"UnsupportedForm: an unknown out-of-range policy"};
  std::vector<J> body = cell;
  for (int d = (int)r - 1; d >= 0; --d) body = {s_for(r + d, int_(0), loc((uint32_t)d), int_(1), body)};
  auto elem = [&](uint32_t k) { return k == index ? EK(idx) : EK(dtype); };
  std::vector<J> params;
  for (uint32_t k = 0; k < n; ++k) params.push_back(param_buffer("in" + std::to_string(k), elem(k), "Read", rank));
  params.push_back(param_buffer("out", EK(dtype), "Write", rank));
  for (uint32_t d = 0; d < r; ++d) params.push_back(param_scalar("n" + std::to_string(d), "I32", d));
  params.push_back(param_scalar("src_extent", EK(idx), extent));
  std::vector<J> locals;
  for (uint32_t i = 0; i < 2 * r; ++i) locals.push_back(local_decl("I32"));
  for (uint32_t k = 0; k < n; ++k) locals.push_back(local_decl(elem(k)));
  locals.push_back(local_decl(EK(idx)));  // src_extent
  locals.push_back(local_decl(EK(idx)));  // clamped index
  J k = kernel_fn(name, EK(dtype), params, locals, body, J::null(), {});
  if (block || grid) grid_stride(k, block, grid);
  return k;
}

// lift_elementwise_opdef (kernel_lift.rs:96-130) and lift_elementwise_opdef_launched (:145-153):
// n inputs loaded at the loop counters into locals 2r..2r+n (input k through its axis permutation
// perms[k] when given: the counter of iteration axis d is the coordinate on the input's axis
// perms[k][d], counter_place :315-324), then `body` with Input(k) bound to those locals stored at
// the counters; the loops nest axis 0 outermost.  The signature (elementwise_signature :328-343):
// the inputs, the output, one I32 extent per axis; locals: the extents, the counters, one loaded
// value per input.  Launched by grid_stride.
J lift_elementwise(const std::string& name, int32_t dtype, int32_t rank, uint32_t n, const J& body_expr,
                   const std::vector<std::vector<int32_t>>& perms, uint32_t block, uint32_t grid) {
  check_rank(rank);
  if (n < 1 || n > 8) throw Decline{"UnsupportedForm: an elementwise op of 1 to 8 inputs"};
  if (!kind_name(dtype)) throw Decline{"UnsupportedForm: an unknown element kind"};
  check_post(body_expr, 0, (int64_t)n);  // leaves_ok: the inputs and constants only
  const uint32_t r = (uint32_t)rank;
  if (!perms.empty()) {
    // check_plain_with (kernel_lift.rs:380-390): one view per input, each a permutation of the axes.
    if (perms.size() != n) throw Decline{"UnsupportedForm: an ill-formed view"};
    for (const auto& p : perms) {
      if (p.size() != r) throw Decline{"UnsupportedForm: an ill-formed view"};
      uint32_t seen = 0;
      for (int32_t a : p) {
        if (a < 0 || a >= rank || ((seen >> a) & 1u)) throw Decline{"UnsupportedForm: an ill-formed view"};
        seen |= 1u << a;
      }
    }
  }
  auto counters = [&](uint32_t buffer, const std::vector<int32_t>* perm) {
    std::vector<J> c(r);
    for (uint32_t d = 0; d < r; ++d) c[perm ? (uint32_t)(*perm)[d] : d] = loc(r + d);
    return p_logical(buffer, c);
  };
  std::vector<J> inner;
  for (uint32_t k = 0; k < n; ++k) inner.push_back(s_load(2 * r + k, counters(k, perms.empty() ? nullptr : &perms[k])));
  const J value = map_leaves(body_expr, [&](const J& x, J& o) {
    if (x.t == J::Obj && x.o.size() == 1 && x.o[0].first == "Input") {
      o = loc(2 * r + (uint32_t)leaf_index(x));
      return true;
    }
    return false;
  });
  inner.push_back(s_store(counters(n, nullptr), value));
  std::vector<J> body = inner;
  for (int d = (int)r - 1; d >= 0; --d) body = {s_for(r + d, int_(0), loc((uint32_t)d), int_(1), body)};
  std::vector<J> params, locals;
  for (uint32_t k = 0; k < n; ++k) params.push_back(param_buffer("in" + std::to_string(k), EK(dtype), "Read", rank));
  params.push_back(param_buffer("out", EK(dtype), "Write", rank));
  for (uint32_t d = 0; d < r; ++d) params.push_back(param_scalar("n" + std::to_string(d), "I32", d));
  for (uint32_t i = 0; i < 2 * r; ++i) locals.push_back(local_decl("I32"));
  for (uint32_t k = 0; k < n; ++k) locals.push_back(local_decl(EK(dtype)));
  J k = kernel_fn(name, EK(dtype), params, locals, body, J::null(), {});
  if (block || grid) grid_stride(k, block, grid);
  return k;
}

// The fused row fold this backend authors for the softmax prologue: out0[r] and out1[r] fold
// row r of a rank-2 input once, each exactly as a serial lifted reduction folds it (kept axis
// outer, reduced axis ascending, f64 accumulator for a float, Max/Min with the NaN rule, one
// cast down at each store).  Launched: rows grid-strided, one thread per row.
J row_reduce2(const std::string& name, int32_t dtype, int32_t op0, int32_t op1, uint32_t block, uint32_t grid) {
  check_accumulated(dtype, op0, "a reduction");
  check_accumulated(dtype, op1, "a reduction");
  if (op0 > UNP_OP_MEAN || op1 > UNP_OP_MEAN)
    throw Decline{"UnsupportedForm: the fused row fold takes Sum, Prod, Max, Min and Mean"};
  const Shape sh(dtype, 2, 0);
  const uint32_t x = 4, a0 = 5, h0 = 6, a1 = 7, h1 = 8, v = 9;
  auto stored = [&](int32_t op, uint32_t acc) {
    J e = loc(acc);
    if (op == UNP_OP_MEAN) e = e_div(e, widen(loc(1), "F64"));
    return (dtype == UNP_F64 || sh.is_int()) ? e : widen(e, EK(dtype));
  };
  std::vector<J> inner = {s_load(x, p_logical(0, {loc(2), loc(3)})), s_let(v, sh.up(loc(x)))};
  for (auto& s : fold_step(op0, a0, h0, v, sh.is_int())) inner.push_back(s);
  for (auto& s : fold_step(op1, a1, h1, v, sh.is_int())) inner.push_back(s);
  std::vector<J> row = {s_let(a0, sh.fold_identity(op0)), s_let(h0, int_(0)), s_let(a1, sh.fold_identity(op1)),
                        s_let(h1, int_(0)), s_for(3, int_(0), loc(1), int_(1), inner),
                        s_store(p_logical(1, {loc(2)}), stored(op0, a0)), s_store(p_logical(2, {loc(2)}), stored(op1, a1))};
  std::vector<J> body = {s_for(2, int_(0), loc(0), int_(1), row)};
  std::vector<J> params = {param_buffer("in0", EK(dtype), "Read", 2), param_buffer("out0", EK(dtype), "Write", 1),
                           param_buffer("out1", EK(dtype), "Write", 1), param_scalar("n0", "I32", 0),
                           param_scalar("n1", "I32", 1)};
  std::vector<J> locals = {local_decl("I32"), local_decl("I32"), local_decl("I32"), local_decl("I32"),
                           local_decl(EK(dtype)), local_decl(sh.acc_ty()), local_decl("I32"), local_decl(sh.acc_ty()),
                           local_decl("I32"), local_decl(sh.acc_ty())};
  J k = kernel_fn(name, EK(dtype), params, locals, body, J::null(), {});
  if (block || grid) grid_stride(k, block, grid);
  return k;
}

// The sub-byte dequant this backend authors (the reference has no dequant lift; this follows
// the dequant-GEMM fixture, crates/unpopped/tests/support/dequant.rs:58-143): for row r and
// column c of a rows x cols matrix, load the 4-bit weight (element r * cols + c of a flat
// U4/I4 buffer), the zero point and the f16 scale of group g (element r * ng + g, ng = ceil(cols
// / G), found by counting since the kernel integer subset has no division), widen the sub-byte
// values to I32 first (kernel_subbyte_load.rs:206-212), subtract, cast to F32, multiply by the
// scale cast to F32, and store the product cast to Bf16 with round-to-nearest-even.  The group
// index advances with an in-group counter.  Launched: rows grid-strided, one thread per row.
J dequant4(const std::string& name, int32_t qk, int32_t zk, int32_t group, uint32_t block, uint32_t grid) {
  if ((qk != UNP_U4 && qk != UNP_I4) || (zk != UNP_U4 && zk != UNP_I4))
    throw Decline{"UnsupportedForm: dequant weights and zero points are U4 or I4"};
  if (group < 1) throw Decline{"UnsupportedForm: a dequant group of zero columns"};
  const uint32_t R = 2, Cc = 3, NG = 4, G = 5, J_ = 6, Q = 7, Z = 8, S = 9, D = 10, F = 11;
  J e = e_add(e_mul(loc(R), loc(1)), loc(Cc));
  J zi = e_add(e_mul(loc(R), loc(NG)), loc(G));
  std::vector<J> inner = {
      s_load(Q, p_logical(0, {e})),
      s_load(Z, p_logical(2, {zi})),
      s_load(S, p_logical(1, {zi})),
      s_let(D, e_sub(e_cast(loc(Q), "I32"), e_cast(loc(Z), "I32"))),
      s_let(F, e_mul(e_cast(loc(D), "F32"), e_cast(loc(S), "F32"))),
      s_store(p_logical(3, {e}), e_cast(loc(F), "Bf16")),
      s_assign(J_, e_add(loc(J_), int_(1))),
      s_if(e_bin("CmpEq", loc(J_), int_(group)), {s_assign(J_, int_(0)), s_assign(G, e_add(loc(G), int_(1)))}, {}),
  };
  std::vector<J> row = {
      s_let(NG, int_(0)),
      s_while(e_bin("CmpLt", e_mul(loc(NG), int_(group)), loc(1)), {s_assign(NG, e_add(loc(NG), int_(1)))}),
      s_let(G, int_(0)),
      s_let(J_, int_(0)),
      s_for(Cc, int_(0), loc(1), int_(1), inner),
  };
  std::vector<J> body = {s_for(R, int_(0), loc(0), int_(1), row)};
  std::vector<J> params = {param_buffer("w", EK(qk), "Read", 1), param_buffer("scale", "F16", "Read", 1),
                           param_buffer("zero", EK(zk), "Read", 1), param_buffer("out", "Bf16", "Write", 1),
                           param_scalar("n0", "I32", 0), param_scalar("n1", "I32", 1)};
  std::vector<J> locals = {local_decl("I32"), local_decl("I32"), local_decl("I32"), local_decl("I32"),
                           local_decl("I32"), local_decl("I32"), local_decl("I32"), local_decl(EK(qk)),
                           local_decl(EK(zk)), local_decl("F16"), local_decl("I32"), local_decl("F32")};
  J k = kernel_fn(name, "F32", params, locals, body, J::null(), {});
  if (block || grid) grid_stride(k, block, grid);
  return k;
}

// The dequantizing GEMM of tests/support/dequant.rs:107-181 with the extents as scalars and int8
// activations: for each row and column, the groups counted without division (as the dequant
// kernel above), then `acc += (widen(w) - zero) * scale * widen(x)` over k, every operation an I32
// that wraps, and one store.
J dequant_gemm(const std::string& name, int32_t wk, int32_t xk, int32_t group, uint32_t block, uint32_t grid) {
  if (wk != UNP_U4 && wk != UNP_I4) throw Decline{"UnsupportedForm: dequant-GEMM weights are U4 or I4"};
  if (xk != UNP_I32 && xk != UNP_I8) throw Decline{"UnsupportedForm: dequant-GEMM activations are I32 or I8"};
  if (group < 1) throw Decline{"UnsupportedForm: a dequant group of zero columns"};
  const uint32_t Rn = 0, Kn = 1, Cn = 2, R = 3, Cc = 4, NG = 5, G = 6, KK = 7, K = 8, ACC = 9, W = 10, Z = 11, S = 12,
                 X = 13;
  const J gi = e_add(e_mul(loc(R), loc(NG)), loc(G));
  std::vector<J> step = {
      s_load(W, p_logical(0, {e_add(e_mul(loc(R), loc(Kn)), loc(K))})),
      s_load(Z, p_logical(1, {gi})),
      s_load(S, p_logical(2, {gi})),
      s_load(X, p_logical(3, {e_add(e_mul(loc(K), loc(Cn)), loc(Cc))})),
      s_assign(ACC, e_add(loc(ACC), e_mul(e_mul(e_sub(e_cast(loc(W), "I32"), loc(Z)), loc(S)), e_cast(loc(X), "I32")))),
      s_assign(KK, e_add(loc(KK), int_(1))),
      s_if(e_bin("CmpEq", loc(KK), int_(group)), {s_assign(KK, int_(0)), s_assign(G, e_add(loc(G), int_(1)))}, {}),
  };
  std::vector<J> col = {s_let(ACC, int_(0)), s_let(G, int_(0)), s_let(KK, int_(0)),
                        s_for(K, int_(0), loc(Kn), int_(1), step),
                        s_store(p_logical(4, {e_add(e_mul(loc(R), loc(Cn)), loc(Cc))}), loc(ACC))};
  std::vector<J> row = {
      s_let(NG, int_(0)),
      s_while(e_bin("CmpLt", e_mul(loc(NG), int_(group)), loc(Kn)), {s_assign(NG, e_add(loc(NG), int_(1)))}),
      s_for(Cc, int_(0), loc(Cn), int_(1), col),
  };
  std::vector<J> body = {s_for(R, int_(0), loc(Rn), int_(1), row)};
  std::vector<J> params = {param_buffer("w", EK(wk), "Read", 1),   param_buffer("zero", "I32", "Read", 1),
                           param_buffer("scale", "I32", "Read", 1), param_buffer("x", EK(xk), "Read", 1),
                           param_buffer("out", "I32", "Write", 1),  param_scalar("n0", "I32", Rn),
                           param_scalar("n1", "I32", Kn),           param_scalar("n2", "I32", Cn)};
  std::vector<J> locals;
  for (int i = 0; i < 10; ++i) locals.push_back(local_decl("I32"));
  locals.push_back(local_decl(EK(wk)));
  locals.push_back(local_decl("I32"));
  locals.push_back(local_decl("I32"));
  locals.push_back(local_decl(EK(xk)));
  J k = kernel_fn(name, "I32", params, locals, body, J::null(), {});
  if (block || grid) grid_stride(k, block, grid);
  return k;
}

// ---- Access::RowReduce (kernel_lift/row_reduce.rs, kernel_lift/row_reduce_launched.rs) ------

// The payload items of a ScalarExpr node (crates/unpopped/src/ir.rs:235-420) that are
// expressions.  False for a node kind this restatement does not carry.
bool expr_slots(const J& e, std::string& tag, std::vector<size_t>& slots, bool& leaf) {
  leaf = false;
  slots.clear();
  if (e.t != J::Obj || e.o.size() != 1) return false;
  tag = e.o[0].first;
  const J& p = e.o[0].second;
  static const char* const leaves[] = {"Input", "Const", "Param", "Reduced", "Coord", "CoordInt", "ConstInt", "Local",
                                       "Exec"};
  for (const char* l : leaves)
    if (tag == l) {
      leaf = true;
      return true;
    }
  if (p.t != J::Arr) return false;
  const size_t n = p.a.size();
  if (tag == "Add" || tag == "Sub" || tag == "Mul" || tag == "Div") {
    slots = {0, 1};
    return n == 2;
  }
  if (tag == "Unary") {
    slots = {1};
    return n == 2;
  }
  if (tag == "Binary") {
    slots = {1, 2};
    return n == 3;
  }
  if (tag == "Select" || tag == "Fma") {
    slots = {0, 1, 2};
    return n == 3;
  }
  if (tag == "Cast" || tag == "Bitcast" || tag == "Qualified" || tag == "Extract") {
    slots = {0};
    return n == 2;
  }
  if (tag == "Pack") {
    for (size_t i = 0; i < n; ++i) slots.push_back(i);
    return true;
  }
  return false;
}

int64_t leaf_index(const J& e) {
  const J& p = e.o[0].second;
  return p.is_int ? p.i : -1;
}

// bind (kernel_lift/post.rs): `e` rebuilt with `leaf` tried first at every node.
template <class F> J map_leaves(const J& e, const F& leaf) {
  J out;
  if (leaf(e, out)) return out;
  std::string tag;
  std::vector<size_t> slots;
  bool is_leaf;
  if (!expr_slots(e, tag, slots, is_leaf))
    throw Decline{"UnsupportedForm: an expression node outside this backend's vocabulary"};
  if (is_leaf) return e;
  J c = e;
  for (size_t i : slots) c.o[0].second.a[i] = map_leaves(e.o[0].second.a[i], leaf);
  return c;
}

// check_post (kernel_lift/post.rs) and leaves_ok (kernel_lift.rs:397-409): a stage's pre may read
// the stages before it, the epilogue every stage; no Coord, Param, Local or Exec leaf.  An Input
// must name one of the op's inputs.
void check_post(const J& e, int64_t available, int64_t n_inputs) {
  std::string tag;
  std::vector<size_t> slots;
  bool leaf;
  if (!expr_slots(e, tag, slots, leaf))
    throw Decline{"UnsupportedForm: an expression node outside this backend's vocabulary"};
  if (leaf) {
    if (tag == "Reduced" && !(leaf_index(e) >= 0 && leaf_index(e) < available))
      throw Decline{"UnsupportedLeaf: a Reduced of a later stage"};
    if (tag == "Coord" || tag == "CoordInt") throw Decline{"UnsupportedLeaf: Coord"};
    if (tag == "Param") throw Decline{"UnsupportedLeaf: Param"};
    if (tag == "Local") throw Decline{"UnsupportedLeaf: Local"};
    if (tag == "Exec") throw Decline{"UnsupportedLeaf: Exec"};
    if (tag == "Input" && !(leaf_index(e) >= 0 && leaf_index(e) < n_inputs))
      throw Decline{"UnsupportedForm: an Input beyond the op's inputs"};
    return;
  }
  for (size_t i : slots) check_post(e.o[0].second.a[i], available, n_inputs);
}

J input_leaf(uint32_t k) { return var("Input", J::integer(k)); }
J reduced_leaf(uint32_t t) { return var("Reduced", J::integer(t)); }

// check_reduction (kernel_lift.rs:807-831) and check_common: the body reads only the op's inputs
// and no Coord, Param, Local, Exec or Reduced leaf; a fused post reads Reduced(0) and no Input.
void check_reduction_exprs(const J& body, const J* post, uint32_t n_inputs) {
  check_post(body, 0, (int64_t)n_inputs);
  if (post) {
    bool reads_input = false;
    map_leaves(*post, [&](const J& x, J&) {
      if (x.t == J::Obj && x.o.size() == 1 && x.o[0].first == "Input") reads_input = true;
      return false;
    });
    if (reads_input) throw Decline{"UnsupportedLeaf: an Input in a reduction post"};
    check_post(*post, 1, 0);
  }
}

J Shape::subst_inputs(const J& body) const {
  return map_leaves(body, [&](const J& x, J& out) {
    if (x.t == J::Obj && x.o.size() == 1 && x.o[0].first == "Input") {
      out = loc(loaded((uint32_t)leaf_index(x)));
      return true;
    }
    return false;
  });
}

J Shape::stored_value(int32_t rop, const J* post, std::vector<J>& body) const {
  if (!post) return stored(rop);
  body.push_back(s_let(red, stored(rop)));
  return map_leaves(*post, [&](const J& x, J& out) {
    if (x.t == J::Obj && x.o.size() == 1 && x.o[0].first == "Reduced") {
      out = loc(red);
      return true;
    }
    return false;
  });
}

// The local ids of row_reduce.rs's `Row`: extents 0..r, counters r..2r, then per phase (each
// stage, then the epilogue) one loaded local per input, then per stage the F64 accumulator, the
// have flag, the current F64 value and the rounded stage result.
struct Row {
  int32_t dtype;
  uint32_t r, n, stages;
  uint32_t counter(uint32_t d) const { return r + d; }
  uint32_t loaded(uint32_t phase, uint32_t k) const { return 2 * r + phase * n + k; }
  uint32_t stage_base(uint32_t s) const { return 2 * r + (stages + 1) * n + 4 * s; }
  J up(J e) const { return dtype == UNP_F64 ? e : widen(std::move(e), "F64"); }
  J down(J e) const { return dtype == UNP_F64 ? e : widen(std::move(e), EK(dtype)); }
  std::vector<J> counters() const {
    std::vector<J> c;
    for (uint32_t d = 0; d < r; ++d) c.push_back(loc(counter(d)));
    return c;
  }
  J for_lead(uint32_t d, std::vector<J> inner) const { return s_for(counter(d), int_(0), loc(d), int_(1), std::move(inner)); }
  J bind(const J& e, uint32_t phase) const {
    return map_leaves(e, [&](const J& x, J& out) {
      if (x.t != J::Obj || x.o.size() != 1) return false;
      if (x.o[0].first == "Input") {
        out = loc(loaded(phase, (uint32_t)leaf_index(x)));
        return true;
      }
      if (x.o[0].first == "Reduced") {
        out = loc(stage_base((uint32_t)leaf_index(x)) + 3);
        return true;
      }
      return false;
    });
  }
  std::vector<J> loads(uint32_t phase) const {
    std::vector<J> v;
    for (uint32_t k = 0; k < n; ++k) v.push_back(s_load(loaded(phase, k), p_logical(k, counters())));
    return v;
  }
  // One stage: fold the row into an F64 accumulator, then round the finalised value once.
  std::vector<J> stage(uint32_t s, const J& pre, int32_t op) const {
    const uint32_t base = stage_base(s), acc = base, have = base + 1, val = base + 2, red = base + 3;
    std::vector<J> inner = loads(s);
    inner.push_back(s_let(val, up(bind(pre, s))));
    for (auto& st : fold_step(op, acc, have, val, false)) inner.push_back(st);
    J fin = op == UNP_OP_MEAN ? e_div(loc(acc), widen(loc(r - 1), "F64")) : loc(acc);
    return {s_let(acc, up(e_const(op == UNP_OP_PROD ? 1.0 : 0.0))), s_let(have, int_(0)), for_lead(r - 1, inner),
            s_let(red, down(fin))};
  }
  J epilogue(const J& epi) const {
    std::vector<J> inner = loads(stages);
    inner.push_back(s_store(p_logical(n, counters()), bind(epi, stages)));
    return for_lead(r - 1, inner);
  }
  void signature(std::vector<J>& params, std::vector<J>& locals) const {
    params.clear();
    for (uint32_t k = 0; k < n; ++k) params.push_back(param_buffer("in" + std::to_string(k), EK(dtype), "Read", (int)r));
    params.push_back(param_buffer("out", EK(dtype), "Write", (int)r));
    for (uint32_t d = 0; d < r; ++d) params.push_back(param_scalar("n" + std::to_string(d), "I32", d));
    locals.clear();
    for (uint32_t i = 0; i < 2 * r; ++i) locals.push_back(local_decl("I32"));
    for (uint32_t i = 0; i < (stages + 1) * n; ++i) locals.push_back(local_decl(EK(dtype)));
    for (uint32_t s = 0; s < stages; ++s) {
      locals.push_back(local_decl("F64"));
      locals.push_back(local_decl("I32"));
      locals.push_back(local_decl("F64"));
      locals.push_back(local_decl(EK(dtype)));
    }
  }
};

// check_row_reduce (row_reduce.rs:51-70).
void check_row_reduce(const RowReduceSpec& sp) {
  if (sp.dtype != UNP_F32 && sp.dtype != UNP_F64) throw Decline{"UnsupportedForm: a non-float row reduction"};
  if (sp.ops.empty()) throw Decline{"UnsupportedForm: an empty stage list"};
  if (sp.ops.size() != sp.pres.size()) throw Decline{"UnsupportedForm: a stage without its pre expression"};
  check_rank(sp.rank);
  if (sp.n_inputs < 1) throw Decline{"UnsupportedForm: a row reduction with no input"};
  for (size_t s = 0; s < sp.ops.size(); ++s) {
    if (!reduce_op_name(sp.ops[s])) throw Decline{"UnsupportedForm: a reduce op outside Sum, Prod, Max, Min and Mean"};
    check_post(sp.pres[s], (int64_t)s, sp.n_inputs);
  }
  check_post(sp.epilogue, (int64_t)sp.ops.size(), sp.n_inputs);
}

// The block tree of block_reduce.rs's `Fold` (publish, rounds) over the accumulator `acc`,
// the have flag `have`, the partner value `val` and the partner's flag `partner_have`.
std::vector<J> fold_publish(int32_t rop, uint32_t acc, uint32_t have) {
  std::vector<J> v = {s_store(p_alloc(0, as_i32(thread())), loc(acc))};
  if (rop == UNP_OP_MAX || rop == UNP_OP_MIN) v.push_back(s_store(p_alloc(1, as_i32(thread())), loc(have)));
  return v;
}
std::vector<J> fold_rounds(int32_t rop, uint32_t block, uint32_t acc, uint32_t have, uint32_t val,
                           uint32_t partner_have, bool is_int) {
  const bool flag = rop == UNP_OP_MAX || rop == UNP_OP_MIN;
  std::vector<J> out;
  for (uint32_t s = block / 2; s > 0; s /= 2) {
    const J partner = as_i32(e_add(thread(), uconst(s)));
    std::vector<J> rb = {s_load(val, p_alloc(0, partner))};
    const std::vector<J> combine = fold_step(rop, acc, have, val, is_int);
    if (flag) {
      rb.push_back(s_load(partner_have, p_alloc(1, partner)));
      rb.push_back(s_if(loc(partner_have), combine, {}));
    } else {
      for (auto& c : combine) rb.push_back(c);
    }
    for (auto& p : fold_publish(rop, acc, have)) rb.push_back(p);
    out.push_back(s_if(e_bin("CmpLt", thread(), uconst(s)), rb, {}));
    out.push_back(s_barrier());
  }
  return out;
}

// A loop statement with its start and step replaced (row_reduce_launched.rs `strided`,
// `block_stride_outermost`).
void restride(J& for_stmt, J start, J step) {
  J& f = for_stmt.o[0].second;
  for (auto& kv : f.o) {
    if (kv.first == "start") kv.second = start;
    if (kv.first == "step") kv.second = step;
  }
}

// lift_row_reduce_opdef (row_reduce.rs:31-49) and lift_row_reduce_opdef_launched
// (row_reduce_launched.rs:47-86).
J lift_row_reduce(const std::string& name, const RowReduceSpec& sp, uint32_t block, uint32_t grid) {
  const bool launched = block || grid;
  if (launched && (grid == 0 || !pow2(block))) throw Decline{"BadLaunch"};
  check_row_reduce(sp);
  const Row w{sp.dtype, (uint32_t)sp.rank, (uint32_t)sp.n_inputs, (uint32_t)sp.ops.size()};
  std::vector<J> params, locals;
  w.signature(params, locals);
  std::vector<J> row;
  if (!launched) {
    for (uint32_t s = 0; s < w.stages; ++s)
      for (auto& st : w.stage(s, sp.pres[s], sp.ops[s])) row.push_back(st);
    row.push_back(w.epilogue(sp.epilogue));
    std::vector<J> body = row;
    for (int d = (int)w.r - 2; d >= 0; --d) body = {w.for_lead((uint32_t)d, body)};
    return kernel_fn(name, EK(sp.dtype), params, locals, body, J::null(), {});
  }
  for (int32_t op : sp.ops)
    if (op == UNP_OP_PROD)
      throw Decline{"UnsupportedForm: a Prod stage in a launched row reduction (a float product is not "
                    "order-independent, and no bound is declared)"};
  if (w.r < 2) throw Decline{"UnsupportedForm: a launched row reduction needs a leading axis to stride blocks over"};
  const J tid = as_i32(thread());
  const J bdim = as_i32(e_exec("BlockDim", 0));
  const uint32_t partner_have = w.stage_base(w.stages);
  for (uint32_t s = 0; s < w.stages; ++s) {
    const uint32_t base = w.stage_base(s);
    std::vector<J> v = w.stage(s, sp.pres[s], sp.ops[s]);
    const J rounded = v.back().o[0].second.get("init") ? *v.back().o[0].second.get("init") : J::null();
    v.pop_back();
    J fold_loop = v.back();
    v.pop_back();
    restride(fold_loop, tid, bdim);
    v.push_back(fold_loop);
    for (auto& st : fold_publish(sp.ops[s], base, base + 1)) v.push_back(st);
    v.push_back(s_barrier());
    for (auto& st : fold_rounds(sp.ops[s], block, base, base + 1, base + 2, partner_have, false)) v.push_back(st);
    v.push_back(s_if(e_bin("CmpEq", thread(), uconst(0)), {s_store(p_alloc(2, int_(s)), rounded)}, {}));
    v.push_back(s_barrier());
    v.push_back(s_load(base + 3, p_alloc(2, int_(s))));
    for (auto& st : v) row.push_back(st);
  }
  J epi = w.epilogue(sp.epilogue);
  restride(epi, tid, bdim);
  row.push_back(epi);
  std::vector<J> body = row;
  for (int d = (int)w.r - 2; d >= 0; --d) body = {w.for_lead((uint32_t)d, body)};
  restride(body[0], as_i32(e_exec("BlockIdx", 0)), as_i32(e_exec("GridDim", 0)));
  locals.push_back(local_decl("I32"));  // the partner's have flag
  std::vector<J> allocs = {alloc_shared("partial", "F64", block), alloc_shared("partial_have", "I32", block),
                           alloc_shared("stage_result", EK(sp.dtype), w.stages)};
  return kernel_fn(name, EK(sp.dtype), params, locals, body, launch_shape(block, grid), allocs);
}

// Undo Row::bind: the locals of phase `phase`'s loads back to Input(k), stage results back to
// Reduced(t).  False when the expression reads any other local.
bool unbind(const Row& w, const J& e, uint32_t phase, J& out) {
  bool ok = true;
  try {
    out = map_leaves(e, [&](const J& x, J& o) {
      if (x.t != J::Obj || x.o.size() != 1 || x.o[0].first != "Local") return false;
      const int64_t l = leaf_index(x);
      for (uint32_t k = 0; k < w.n; ++k)
        if (l == (int64_t)w.loaded(phase, k)) {
          o = var("Input", J::integer(k));
          return true;
        }
      for (uint32_t t = 0; t < w.stages; ++t)
        if (l == (int64_t)w.stage_base(t) + 3) {
          o = var("Reduced", J::integer(t));
          return true;
        }
      ok = false;
      o = x;
      return true;
    });
  } catch (const Decline&) {
    return false;
  }
  return ok;
}

// Depth-first search of a statement list for the first statement `pick` accepts.
template <class F> const J* find_stmt(const J& block, const F& pick) {
  if (block.t != J::Arr) return nullptr;
  for (const J& st : block.a) {
    if (pick(st)) return &st;
    if (st.t != J::Obj || st.o.size() != 1) continue;
    const J& b = st.o[0].second;
    for (const char* key : {"then", "els", "body"}) {
      const J* inner = b.get(key);
      if (inner) {
        const J* f = find_stmt(*inner, pick);
        if (f) return f;
      }
    }
  }
  return nullptr;
}

// ---- recognition -------------------------------------------------------------------------

// Fill the serde defaults a writer may omit (KernelFn: launch, allocs, result, results;
// LaunchShape: cluster, devices, grid_dims; For: unroll), recursively.
void normalize(J& j, bool top) {
  if (j.t == J::Arr) {
    for (auto& x : j.a) normalize(x, false);
    return;
  }
  if (j.t != J::Obj) return;
  auto ensure = [&](const char* key, J v) {
    if (!j.get(key)) j.o.emplace_back(key, std::move(v));
  };
  if (top) {
    ensure("launch", J::null());
    ensure("allocs", J::arr());
    ensure("result", J::null());
    ensure("results", J::arr());
    for (auto& kv : j.o)
      if (kv.first == "launch" && kv.second.t == J::Obj) {
        J& l = kv.second;
        if (!l.get("subgroup")) l.o.emplace_back("subgroup", J::null());
        if (!l.get("cluster")) l.o.emplace_back("cluster", J::null());
        if (!l.get("devices")) l.o.emplace_back("devices", J::integer(1));
        if (!l.get("grid_dims")) l.o.emplace_back("grid_dims", J::null());
      }
  }
  if (j.o.size() == 1 && j.o[0].first == "For" && j.o[0].second.t == J::Obj) {
    J& f = j.o[0].second;
    if (!f.get("unroll")) f.o.emplace_back("unroll", unit("None"));
  }
  for (auto& kv : j.o)
    if (!(top && kv.first == "launch")) normalize(kv.second, false);
}

// ---- local renumbering ----------------------------------------------------------------------
// A KernelFn names its locals by index (LocalId, kernel.rs): the ScalarExpr leaf Local(n) and the
// `local` of Let, Load, Assign, For and a Scalar parameter.  Two kernels that differ only by a
// consistent renumbering of their locals (the locals list permuted to match) are the same kernel.

// Every local-id reference of `j`, each object's keys in sorted order (so that the visit does not
// depend on the order a writer put the keys in).
template <class F>
void visit_local_refs(J& j, F& f) {
  if (j.t == J::Arr) {
    for (auto& x : j.a) visit_local_refs(x, f);
    return;
  }
  if (j.t != J::Obj) return;
  if (j.o.size() == 1 && j.o[0].first == "Local" && j.o[0].second.t == J::Num && j.o[0].second.is_int) {
    f(j.o[0].second);
    return;
  }
  std::vector<size_t> order(j.o.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = i;
  std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return j.o[a].first < j.o[b].first; });
  for (size_t i : order) {
    auto& kv = j.o[i];
    if (kv.first == "local" && kv.second.t == J::Num && kv.second.is_int) f(kv.second);
    else visit_local_refs(kv.second, f);
  }
}

// The references of a KernelFn: its parameters, then its body.
template <class F>
void visit_kernel_locals(J& k, F& f) {
  for (auto& kv : k.o)
    if (kv.first == "params") visit_local_refs(kv.second, f);
  for (auto& kv : k.o)
    if (kv.first == "body") visit_local_refs(kv.second, f);
}

// A JSON value with every object's keys sorted (the same text whatever order a writer used).
J sorted_keys(const J& j) {
  J c = j;
  if (c.t == J::Arr) {
    for (auto& x : c.a) x = sorted_keys(x);
  } else if (c.t == J::Obj) {
    for (auto& kv : c.o) kv.second = sorted_keys(kv.second);
    std::sort(c.o.begin(), c.o.end(), [](const std::pair<std::string, J>& a, const std::pair<std::string, J>& b) {
      return a.first < b.first;
    });
  }
  return c;
}

size_t local_count(const J& k) {
  const J* l = k.get("locals");
  return (l && l->t == J::Arr) ? l->a.size() : 0;
}

// The canonical numbering of k's locals: in order of first reference, then the unreferenced ones
// ordered by their declarations (which alone tell them apart).  False when a reference names no
// declared local.
bool canonical_order(const J& k, std::vector<int64_t>& to) {
  const size_t m = local_count(k);
  to.assign(m, -1);
  int64_t next = 0;
  bool ok = true;
  J copy = k;
  auto first = [&](J& id) {
    if (id.i < 0 || (size_t)id.i >= m) {
      ok = false;
      return;
    }
    if (to[(size_t)id.i] < 0) to[(size_t)id.i] = next++;
  };
  visit_kernel_locals(copy, first);
  std::vector<std::pair<std::string, size_t>> rest;
  const J* decls = k.get("locals");
  for (size_t i = 0; i < m; ++i)
    if (to[i] < 0) rest.emplace_back(kir::write(sorted_keys(decls->a[i])), i);
  std::stable_sort(rest.begin(), rest.end(),
                   [](const std::pair<std::string, size_t>& a, const std::pair<std::string, size_t>& b) {
                     return a.first < b.first;
                   });
  for (const auto& r : rest) to[r.second] = next++;
  return ok;
}

// k with local i renamed to[i] (a permutation) and its locals list permuted to match.
J renumbered(const J& k, const std::vector<int64_t>& to) {
  J c = k;
  auto rename = [&](J& id) {
    if (id.i >= 0 && (size_t)id.i < to.size()) id.i = to[(size_t)id.i];
  };
  visit_kernel_locals(c, rename);
  for (auto& kv : c.o)
    if (kv.first == "locals" && kv.second.t == J::Arr && kv.second.a.size() == to.size()) {
      std::vector<J> perm(to.size());
      for (size_t i = 0; i < to.size(); ++i) perm[(size_t)to[i]] = kv.second.a[i];
      kv.second.a = std::move(perm);
    }
  return c;
}

// k in its canonical numbering (unchanged when a reference names no declared local).
J canonical(const J& k) {
  std::vector<int64_t> to;
  return canonical_order(k, to) ? renumbered(k, to) : k;
}

// The canonical kernel `kc` renumbered into the numbering of `proto`: the kernel as the lift that
// produced `proto` would number it, when the two share a statement skeleton (the expressions a
// caller supplies read only locals defined before them, so they do not move a first reference).
bool into_numbering_of(const J& proto, const J& kc, J& out) {
  std::vector<int64_t> to;
  if (!canonical_order(proto, to) || to.size() != local_count(kc)) return false;
  std::vector<int64_t> back(to.size());
  for (size_t i = 0; i < to.size(); ++i) back[(size_t)to[i]] = (int64_t)i;
  out = renumbered(kc, back);
  return true;
}

struct ParamInfo {
  bool buffer = false;
  int32_t elem = -1;
  std::string role;
  int rank = -1;
};

bool read_params(const J& k, std::vector<ParamInfo>& out) {
  const J* ps = k.get("params");
  if (!ps || ps->t != J::Arr) return false;
  for (const J& p : ps->a) {
    const J* kind = p.get("kind");
    if (!kind || kind->t != J::Obj || kind->o.size() != 1) return false;
    ParamInfo pi;
    const J& body = kind->o[0].second;
    if (kind->o[0].first == "Buffer") {
      pi.buffer = true;
      const J* e = body.get("elem");
      const J* role = body.get("role");
      const J* rank = body.get("rank");
      if (!e || e->t != J::Str || !role || role->t != J::Str) return false;
      pi.elem = kind_from_name(e->s);
      pi.role = role->s;
      pi.rank = (rank && rank->t == J::Num) ? (int)rank->i : -1;
    } else if (kind->o[0].first == "Scalar") {
      const J* t = body.get("ty");
      if (!t || t->t != J::Str) return false;
      pi.elem = kind_from_name(t->s);
    } else {
      return false;
    }
    out.push_back(pi);
  }
  return true;
}

}  // namespace

int32_t recognize_kernel(const std::string& text, Recognized& out, std::string& why) {
  J k;
  if (!kir::parse(text, k, why)) {
    why = "kernel JSON: " + why;
    return UNP_PARSE_ERROR;
  }
  if (k.t != J::Obj || !k.get("name") || k.get("name")->t != J::Str || !k.get("compute") || !k.get("body")) {
    why = "not a KernelFn: expected an object with name, compute, params, locals and body";
    return UNP_PARSE_ERROR;
  }
  normalize(k, true);
  const J kc = canonical(k);  // compared in the canonical numbering of locals
  const std::string name = k.get("name")->s;
  std::vector<ParamInfo> ps;
  if (!read_params(k, ps)) {
    why = "not a KernelFn: malformed params";
    return UNP_PARSE_ERROR;
  }
  uint32_t block = 0, grid = 0;
  const J* launch = k.get("launch");
  if (launch->t == J::Obj) {
    const J* b = launch->get("block");
    const J* g = launch->get("grid");
    if (b && b->t == J::Arr && !b->a.empty() && b->a[0].is_int) block = (uint32_t)b->a[0].i;
    if (g && g->t == J::Arr && !g->a.empty() && g->a[0].is_int) grid = (uint32_t)g->a[0].i;
    if (!block || !grid) {
      why = "a launch shape with a zero block or grid";
      return UNP_UNSUPPORTED_KERNEL;
    }
  }
  out.name = name;
  out.launch = *launch;
  out.params = *k.get("params");
  auto matches = [&](const J& cand) {
    J c = cand;
    for (auto& kv : c.o)
      if (kv.first == "name") kv.second = J::str(name);
    return canonical(c) == kc;
  };
  auto attempt = [&](auto&& make) {
    try {
      return matches(make());
    } catch (const Decline&) {
      return false;
    }
  };
  const size_t np = ps.size();
  // Reduction or scan: in0..in(n-1) Read (rank r, one dtype), out Write, then r I32 extents.
  // A reduction's body is read back from its `val` Let (the up-cast stripped, the loaded locals
  // unbound to Input(k)) and a fused post from the output store (Local(red) unbound to
  // Reduced(0)); each candidate is re-lifted with them and compared as a whole.
  size_t nin = 0;
  if (np >= 3 && ps[0].buffer && ps[0].role == "Read" && ps[0].rank >= 1 && (size_t)ps[0].rank + 2 <= np) {
    nin = np - 1 - (size_t)ps[0].rank;
    for (size_t i = 0; i < nin && nin; ++i)
      if (!ps[i].buffer || ps[i].role != "Read" || ps[i].rank != ps[0].rank || ps[i].elem != ps[0].elem) nin = 0;
    if (nin && !(ps[nin].buffer && ps[nin].role == "Write")) nin = 0;
    for (size_t i = nin + 1; nin && i < np; ++i)
      if (ps[i].buffer) nin = 0;
  }
  if (nin >= 1 && nin <= 8) {
    const int32_t dt = ps[0].elem, r = ps[0].rank, orank = ps[nin].rank;
    const uint32_t n = (uint32_t)nin;
    // Elementwise (kernel_lift.rs:96-153): the body read back from the output store (the loaded
    // locals unbound to Input(k)) and each input's permutation from its load's coordinates, in the
    // lift's numbering of locals; the lift re-run with them and compared as a whole.
    if (orank == r && ps[nin].elem == dt) {
      auto ew_extract = [&](const J& kk, J& body, std::vector<std::vector<int32_t>>& perms) {
        const J& kb = *kk.get("body");
        const J* store = find_stmt(kb, [&](const J& x) {
          const J* st = x.get("Store");
          const J* pl = st ? st->get("place") : nullptr;
          const J* lg = pl ? pl->get("Logical") : nullptr;
          return lg && lg->get("buffer") && lg->get("buffer")->is_int && lg->get("buffer")->i == (int64_t)n;
        });
        if (!store) return false;
        bool ok = true;
        try {
          body = map_leaves(*store->get("Store")->get("value"), [&](const J& x, J& o) {
            if (x.t != J::Obj || x.o.size() != 1 || x.o[0].first != "Local") return false;
            const int64_t l = leaf_index(x);
            if (l >= 2 * (int64_t)r && l < 2 * (int64_t)r + (int64_t)n) {
              o = input_leaf((uint32_t)(l - 2 * r));
            } else {
              ok = false;
              o = x;
            }
            return true;
          });
        } catch (const Decline&) {
          return false;
        }
        if (!ok) return false;
        perms.assign(n, std::vector<int32_t>());
        bool any = false;
        for (uint32_t kk2 = 0; kk2 < n; ++kk2) {
          const J* ld = find_stmt(kb, [&](const J& x) {
            const J* l = x.get("Load");
            return l && l->get("local") && l->get("local")->is_int && l->get("local")->i == (int64_t)(2 * r + kk2);
          });
          const J* pl = ld ? ld->get("Load")->get("place") : nullptr;
          const J* lg = pl ? pl->get("Logical") : nullptr;
          const J* cs = lg ? lg->get("coords") : nullptr;
          if (!cs || cs->t != J::Arr || cs->a.size() != (size_t)r) return false;
          std::vector<int32_t> p((size_t)r, -1);
          for (int32_t a = 0; a < r; ++a) {
            const J& c = cs->a[(size_t)a];
            if (c.t != J::Obj || c.o.size() != 1 || c.o[0].first != "Local") return false;
            const int64_t d = leaf_index(c) - r;
            if (d < 0 || d >= r || p[(size_t)d] != -1) return false;
            p[(size_t)d] = a;
          }
          for (int32_t d = 0; d < r; ++d) any = any || p[(size_t)d] != d;
          perms[kk2] = p;
        }
        if (!any) perms.clear();
        return true;
      };
      auto take_elementwise = [&](const J& b, const std::vector<std::vector<int32_t>>& pm) {
        out.form.kind = UNP_FORM_ELEMENTWISE;
        out.form.dtype = dt;
        out.form.rank = r;
        out.ew.n_inputs = (int32_t)n;
        out.ew.body = b;
        out.ew.perms = pm;
        out.lift = block ? "lift_elementwise_opdef_launched" : "lift_elementwise_opdef";
        return UNP_OK;
      };
      J eb, kr;
      std::vector<std::vector<int32_t>> ep;
      if (ew_extract(k, eb, ep) && attempt([&] { return lift_elementwise(name, dt, r, n, eb, ep, block, grid); }))
        return take_elementwise(eb, ep);
      // Locals numbered otherwise: renumbered into the lift's own numbering first (the loads
      // define the loaded locals in input order before the store reads them).
      bool proto_ok = true;
      J proto;
      try {
        proto = lift_elementwise(name, dt, r, n, input_leaf(0), {}, block, grid);
      } catch (const Decline&) {
        proto_ok = false;
      }
      if (proto_ok && into_numbering_of(proto, kc, kr) && ew_extract(kr, eb, ep) &&
          attempt([&] { return lift_elementwise(name, dt, r, n, eb, ep, block, grid); }))
        return take_elementwise(eb, ep);
    }
    // The pre-map body read back from the `val` Let (the up-cast stripped, the loaded locals
    // unbound to Input(k)) and a fused post from the output store (Local(red) unbound to
    // Reduced(0)), in the lift's numbering of locals; false when they read any other local.
    auto extract = [&](const J& kk, J& xbody, J& xpost, bool& has_post) {
      xbody = input_leaf(0);
      xpost = J();
      has_post = false;
      bool exprs_ok = true;
      const uint32_t val = 2 * (uint32_t)r + n + 2, red = val + 1;
      auto unbind_locals = [&](const J& e, J& o) {
        bool ok = true;
        try {
          o = map_leaves(e, [&](const J& x, J& out2) {
            if (x.t != J::Obj || x.o.size() != 1 || x.o[0].first != "Local") return false;
            const int64_t l = leaf_index(x);
            if (l >= 2 * (int64_t)r && l < 2 * (int64_t)r + (int64_t)n) out2 = input_leaf((uint32_t)(l - 2 * r));
            else if (l == (int64_t)red) out2 = reduced_leaf(0);
            else {
              ok = false;
              out2 = x;
            }
            return true;
          });
        } catch (const Decline&) {
          return false;
        }
        return ok;
      };
      const J& kb = *kk.get("body");
      const J* let = find_stmt(kb, [&](const J& x) {
        const J* l = x.get("Let");
        return l && l->get("local") && l->get("local")->is_int && l->get("local")->i == (int64_t)val;
      });
      if (let) {
        J init = *let->get("Let")->get("init");
        if (dt == UNP_F32) {
          const J* c = init.get("Cast");
          if (c && c->t == J::Arr && c->a.size() == 2) {
            J operand = c->a[0];
            init = std::move(operand);
          } else {
            exprs_ok = false;
          }
        }
        if (exprs_ok && !unbind_locals(init, xbody)) exprs_ok = false;
      }
      const J* store = find_stmt(kb, [&](const J& x) {
        const J* st = x.get("Store");
        const J* pl = st ? st->get("place") : nullptr;
        const J* lg = pl ? pl->get("Logical") : nullptr;
        return lg && lg->get("buffer") && lg->get("buffer")->is_int && lg->get("buffer")->i == (int64_t)n;
      });
      if (exprs_ok && store) {
        const J& v = *store->get("Store")->get("value");
        bool reads_red = false;
        map_leaves(v, [&](const J& x, J&) {
          if (x.t == J::Obj && x.o.size() == 1 && x.o[0].first == "Local" && leaf_index(x) == (int64_t)red)
            reads_red = true;
          return false;
        });
        if (reads_red) {
          has_post = unbind_locals(v, xpost);
          if (!has_post) exprs_ok = false;
        }
      }
      return exprs_ok;
    };
    J xbody, xpost;
    bool has_post = false;
    const bool exprs_ok = extract(k, xbody, xpost, has_post);
    auto take_reduction = [&](int32_t op, uint32_t mask, const J& b, const J& p, bool hp) {
      out.form.kind = UNP_FORM_REDUCTION;
      out.form.dtype = dt;
      out.form.rank = r;
      out.form.op0 = op;
      out.form.axes_mask = mask;
      out.rx.n_inputs = (int32_t)n;
      out.rx.body = b;
      out.rx.has_post = hp;
      out.rx.post = p;
      out.rx.plain = n == 1 && b == input_leaf(0) && !hp;
      out.form.reduced_from = r;
      for (int32_t d = r - 1; d >= 0 && ((mask >> d) & 1u); --d) out.form.reduced_from = d;
      out.lift = block ? "lift_reduction_opdef_launched" : "lift_reduction_opdef";
      return UNP_OK;
    };
    auto take_scan = [&](int32_t op, int32_t axis, int ex, int rev, const J& b, const J& p, bool hp) {
      out.form.kind = UNP_FORM_SCAN;
      out.form.dtype = dt;
      out.form.rank = r;
      out.form.op0 = op;
      out.form.exclusive = ex;
      out.form.reverse = rev;
      out.form.axes_mask = axis == r - 1 ? 0u : (1u << axis);
      out.rx.n_inputs = (int32_t)n;
      out.rx.body = b;
      out.rx.has_post = hp;
      out.rx.post = p;
      out.rx.plain = n == 1 && b == input_leaf(0) && !hp;
      out.lift = block ? "lift_scan_opdef_launched" : "lift_scan_opdef";
      return UNP_OK;
    };
    static const int32_t ops[] = {UNP_OP_SUM,    UNP_OP_PROD, UNP_OP_MAX, UNP_OP_MIN, UNP_OP_MEAN,
                                  UNP_OP_MAXNUM, UNP_OP_MINNUM, UNP_OP_AND, UNP_OP_OR, UNP_OP_XOR};
    // Every reduced-axis set whose output rank matches (ReductionShape::new,
    // kernel_lift.rs:854-870), trailing runs first: the reduction most often asked for.
    std::vector<uint32_t> masks;
    for (int32_t from = r - 1; from >= 0; --from) masks.push_back(((1u << r) - 1) & ~((1u << from) - 1));
    for (uint32_t m = 1; m < (1u << r); ++m)
      if (std::find(masks.begin(), masks.end(), m) == masks.end()) masks.push_back(m);
    for (int32_t op : ops) {
      for (uint32_t mask : masks) {
        const int32_t kept = r - __builtin_popcount(mask);
        for (int keep = 0; keep <= 1; ++keep) {
          const int32_t want = keep ? r : kept;
          if (orank != want) continue;
          if (exprs_ok && attempt([&] {
                return lift_reduction(name, dt, r, op, mask, keep, block, grid, n, &xbody, has_post ? &xpost : nullptr);
              }))
            return take_reduction(op, mask, xbody, xpost, has_post);
        }
      }
      if (orank == r && exprs_ok) {
        // The innermost axis first (the only one a launched scan takes), then the others.
        for (int32_t ai = 0; ai < r; ++ai) {
          const int32_t axis = ai == 0 ? r - 1 : ai - 1;
          for (int ex = 0; ex <= 1; ++ex)
            for (int rev = 0; rev <= 1; ++rev)
              if (attempt([&] {
                    return lift_scan(name, dt, r, op, axis, ex, rev, block, grid, n, &xbody, has_post ? &xpost : nullptr);
                  }))
                return take_scan(op, axis, ex, rev, xbody, xpost, has_post);
        }
      }
    }
    // A kernel whose locals are numbered otherwise: renumbered into each candidate skeleton's own
    // numbering (the lift with the plain body, with and without a fused post), its body and post
    // read back there, and the candidate re-lifted with them and compared.
    const J probe_post = e_add(reduced_leaf(0), reduced_leaf(0));
    for (int32_t op : ops)
      for (uint32_t mask : masks) {
        const int32_t kept = r - __builtin_popcount(mask);
        for (int keep = 0; keep <= 1; ++keep) {
          if (orank != (keep ? r : kept)) continue;
          for (int pm = 0; pm <= 1; ++pm) {
            J proto, kr, b, p;
            bool hp = false;
            try {
              proto = lift_reduction(name, dt, r, op, mask, keep, block, grid, n, nullptr, pm ? &probe_post : nullptr);
            } catch (const Decline&) {
              continue;
            }
            if (!into_numbering_of(proto, kc, kr) || !extract(kr, b, p, hp) || hp != (pm == 1)) continue;
            if (attempt([&] { return lift_reduction(name, dt, r, op, mask, keep, block, grid, n, &b, hp ? &p : nullptr); }))
              return take_reduction(op, mask, b, p, hp);
          }
        }
      }
    if (orank == r)
      for (int32_t op : ops)
        for (int32_t axis = r - 1; axis >= 0; --axis)
          for (int ex = 0; ex <= 1; ++ex)
            for (int rev = 0; rev <= 1; ++rev)
              for (int pm = 0; pm <= 1; ++pm) {
                J proto, kr, b, p;
                bool hp = false;
                try {
                  proto = lift_scan(name, dt, r, op, axis, ex, rev, block, grid, n, nullptr, pm ? &probe_post : nullptr);
                } catch (const Decline&) {
                  continue;
                }
                if (!into_numbering_of(proto, kc, kr) || !extract(kr, b, p, hp) || hp != (pm == 1)) continue;
                if (attempt([&] {
                      return lift_scan(name, dt, r, op, axis, ex, rev, block, grid, n, &b, hp ? &p : nullptr);
                    }))
                  return take_scan(op, axis, ex, rev, b, p, hp);
              }
  }
  // Fused row fold: in0 Read rank 2, out0 / out1 Write rank 1, two I32 extents.
  if (np == 5 && ps[0].buffer && ps[0].rank == 2 && ps[1].buffer && ps[2].buffer && !ps[3].buffer && !ps[4].buffer) {
    static const int32_t ops[] = {UNP_OP_SUM, UNP_OP_PROD, UNP_OP_MAX, UNP_OP_MIN, UNP_OP_MEAN};
    for (int32_t a : ops)
      for (int32_t b : ops)
        if (attempt([&] { return row_reduce2(name, ps[0].elem, a, b, block, grid); })) {
          out.form.kind = UNP_FORM_ROW_REDUCE2;
          out.form.dtype = ps[0].elem;
          out.form.rank = 2;
          out.form.op0 = a;
          out.form.op1 = b;
          out.form.reduced_from = 1;
          out.lift = "row_reduce2";
          return UNP_OK;
        }
  }
  // Gather: n inputs (one the integer index), out (Write), r I32 extents, src_extent of the index
  // dtype.  The body is read back from the cell's last store (the loaded locals unbound to
  // Input(k)); each candidate (index slot, data slot, axis, policy) is re-lifted and compared.
  {
    size_t nb = 0;
    while (nb < np && ps[nb].buffer) ++nb;
    const size_t n = nb >= 3 ? nb - 1 : 0;
    const int32_t r = n ? ps[n].rank : 0;
    const bool shape = n >= 2 && n <= 8 && ps[n].role == "Write" && r >= 1 && r <= 8 && np == nb + (size_t)r + 1 &&
                       (ps[np - 1].elem == UNP_I32 || ps[np - 1].elem == UNP_I64 || ps[np - 1].elem == UNP_U32);
    bool sig_ok = shape;
    for (size_t i = nb; sig_ok && i + 1 < np; ++i) sig_ok = ps[i].elem == UNP_I32;
    for (size_t i = 0; sig_ok && i < n; ++i) sig_ok = ps[i].role == "Read" && ps[i].rank == r;
    const int32_t idx = sig_ok ? ps[np - 1].elem : -1, dt = sig_ok ? ps[n].elem : -1;
    static const int32_t pols[] = {UNP_OOB_SKIP, UNP_OOB_ZEROFILL, UNP_OOB_CLAMP};
    // The body of the kernel `kk` in the lift's numbering: the last store to the output.
    auto gather_body = [&](const J& kk, J& body) {
      const J* last = nullptr;
      find_stmt(*kk.get("body"), [&](const J& x) {
        const J* st = x.get("Store");
        const J* pl = st ? st->get("place") : nullptr;
        const J* lg = pl ? pl->get("Logical") : nullptr;
        if (lg && lg->get("buffer") && lg->get("buffer")->is_int && lg->get("buffer")->i == (int64_t)n) last = &x;
        return false;
      });
      if (!last) return false;
      bool ok = true;
      try {
        body = map_leaves(*last->get("Store")->get("value"), [&](const J& x, J& o) {
          if (x.t != J::Obj || x.o.size() != 1 || x.o[0].first != "Local") return false;
          const int64_t l = leaf_index(x);
          if (l >= 2 * (int64_t)r && l < 2 * (int64_t)r + (int64_t)n) o = input_leaf((uint32_t)(l - 2 * r));
          else {
            ok = false;
            o = x;
          }
          return true;
        });
      } catch (const Decline&) {
        return false;
      }
      return ok;
    };
    auto take_gather = [&](uint32_t index, uint32_t data, int32_t axis, int32_t pol, const J& body) {
      out.form.kind = UNP_FORM_GATHER;
      out.form.axes_mask = axis == 0 ? 0u : (1u << axis);
      out.form.dtype = dt;
      out.form.rank = r;
      out.form.index_dtype = idx;
      out.form.oob = pol;
      out.form.data_slot = (int32_t)data;
      out.gx.n_inputs = (int32_t)n;
      out.gx.index_slot = (int32_t)index;
      out.gx.body = body;
      out.gx.plain = n == 2 && body == input_leaf(data);
      out.lift = block ? "lift_gather_opdef_launched" : "lift_gather_opdef";
      return UNP_OK;
    };
    for (int pass = 0; sig_ok && pass < 2; ++pass) {
      for (uint32_t index = 0; index < n; ++index) {
        if (ps[index].elem != idx) continue;
        bool others = true;
        for (uint32_t k = 0; k < n; ++k)
          if (k != index && ps[k].elem != dt) others = false;
        if (!others) continue;
        J body;
        const bool fast_body = pass == 0 && gather_body(k, body);
        if (pass == 0 && !fast_body) continue;
        for (uint32_t data = 0; data < n; ++data) {
          if (data == index) continue;
          for (int32_t axis = 0; axis < r; ++axis)
            for (int32_t pol : pols) {
              if (pass == 1) {
                // Locals numbered otherwise: renumber into the candidate's numbering first.
                J proto, kr;
                try {
                  proto = lift_gather(name, dt, r, idx, axis, pol, block, grid, (uint32_t)n, data, index);
                } catch (const Decline&) {
                  continue;
                }
                if (!into_numbering_of(proto, kc, kr) || !gather_body(kr, body)) continue;
              }
              if (attempt([&] { return lift_gather(name, dt, r, idx, axis, pol, block, grid, (uint32_t)n, data, index, &body); }))
                return take_gather(index, data, axis, pol, body);
            }
        }
      }
    }
  }
  // Dequant: w (U4/I4), scale (F16), zero (U4/I4), out (Bf16), two I32 extents; the group is
  // the constant of the column-group counting loop.
  if (np == 6 && ps[0].buffer && ps[1].buffer && ps[2].buffer && ps[3].buffer && ps[1].elem == UNP_F16 &&
      ps[3].elem == UNP_BF16) {
    int64_t group = -1;
    const J* body = k.get("body");
    // body[0] = For rows { .., While(CmpLt(Mul(ng, G), n1)) .. }
    if (body && body->t == J::Arr && !body->a.empty() && body->a[0].get("For")) {
      const J* rowb = body->a[0].get("For")->get("body");
      if (rowb && rowb->t == J::Arr && rowb->a.size() > 1 && rowb->a[1].get("While")) {
        const J* cond = rowb->a[1].get("While")->get("cond");
        const J* bin = cond ? cond->get("Binary") : nullptr;
        if (bin && bin->t == J::Arr && bin->a.size() == 3) {
          const J* mul = bin->a[1].get("Mul");
          if (mul && mul->t == J::Arr && mul->a.size() == 2) {
            const J* ci = mul->a[1].get("ConstInt");
            if (ci && ci->t == J::Arr && !ci->a.empty() && ci->a[0].is_int) group = ci->a[0].i;
          }
        }
      }
    }
    if (group >= 1 && group <= (1 << 30) &&
        attempt([&] { return dequant4(name, ps[0].elem, ps[2].elem, (int32_t)group, block, grid); })) {
      out.form.kind = UNP_FORM_DEQUANT4;
      out.form.q_kind = ps[0].elem;
      out.form.z_kind = ps[2].elem;
      out.form.group = (int32_t)group;
      out.form.out_kind = UNP_BF16;
      out.lift = "dequant4";
      return UNP_OK;
    }
  }
  // The dequantizing GEMM: w (U4/I4), zero, scale (I32), x (I32/I8) Read, out (I32) Write, three
  // I32 extents; the group read back from the in-group counter's wrap test.
  if (np == 8 && ps[0].buffer && (ps[0].elem == UNP_U4 || ps[0].elem == UNP_I4) && ps[1].buffer &&
      ps[1].elem == UNP_I32 && ps[2].buffer && ps[2].elem == UNP_I32 && ps[3].buffer &&
      (ps[3].elem == UNP_I8 || ps[3].elem == UNP_I32) && ps[4].buffer && ps[4].elem == UNP_I32 &&
      ps[4].role == "Write") {
    int64_t group = 0;
    const J* cmp = find_stmt(*k.get("body"), [&](const J& x) {
      const J* i = x.get("If");
      const J* cond = i ? i->get("cond") : nullptr;
      const J* bin = cond ? cond->get("Binary") : nullptr;
      return bin && bin->t == J::Arr && bin->a.size() == 3 && bin->a[0].t == J::Str && bin->a[0].s == "CmpEq";
    });
    if (cmp) {
      const J* ci = cmp->get("If")->get("cond")->get("Binary")->a[2].get("ConstInt");
      if (ci && ci->t == J::Arr && !ci->a.empty() && ci->a[0].is_int) group = ci->a[0].i;
    }
    if (group >= 1 && group <= (1 << 30) &&
        attempt([&] { return dequant_gemm(name, ps[0].elem, ps[3].elem, (int32_t)group, block, grid); })) {
      out.form.kind = UNP_FORM_DEQUANT_GEMM;
      out.form.q_kind = ps[0].elem;
      out.form.dtype = ps[3].elem;
      out.form.out_kind = UNP_I32;
      out.form.group = (int32_t)group;
      out.lift = "dequant_gemm";
      return UNP_OK;
    }
  }
  // Access::RowReduce: n inputs (Read, rank r), out (Write, rank r), r I32 extents.  The stage
  // count follows from the locals; each stage's pre and the epilogue are read back from the
  // tree (un-binding the loaded and stage-result locals), each stage's fold from its accumulate
  // step, and the candidate is re-lifted and compared as a whole.
  for (size_t n = 1; n + 2 <= np; ++n) {
    const size_t r = np - 1 - n;
    bool shape = ps[n].buffer && ps[n].role == "Write" && (size_t)ps[n].rank == r &&
                 (ps[0].elem == UNP_F32 || ps[0].elem == UNP_F64);
    for (size_t i = 0; shape && i < n; ++i)
      shape = ps[i].buffer && ps[i].role == "Read" && (size_t)ps[i].rank == r && ps[i].elem == ps[0].elem;
    for (size_t i = n + 1; shape && i < np; ++i) shape = !ps[i].buffer && ps[i].elem == UNP_I32;
    if (!shape || r < 1 || r > 8) continue;
    const J* locs = k.get("locals");
    if (!locs || locs->t != J::Arr) continue;
    const int64_t L = (int64_t)locs->a.size() - (block ? 1 : 0) - 2 * (int64_t)r - (int64_t)n;
    if (L <= 0 || L % (int64_t)(n + 4) != 0) continue;
    const uint32_t S = (uint32_t)(L / (int64_t)(n + 4));
    if (S > 8) continue;
    const Row w{ps[0].elem, (uint32_t)r, (uint32_t)n, S};
    RowReduceSpec sp;
    sp.dtype = ps[0].elem;
    sp.rank = (int32_t)r;
    sp.n_inputs = (int32_t)n;
    // Reads the stages' pres, folds and the epilogue back from `kk` (in the lift's numbering of
    // locals) and tries every combination of the candidate folds.
    auto try_row_reduce = [&](const J& kk) {
      const J& body = *kk.get("body");
      sp.pres.clear();
      sp.ops.clear();
      bool ok = true;
      std::vector<std::vector<int32_t>> cand;
      for (uint32_t st = 0; ok && st < S; ++st) {
        const uint32_t val = w.stage_base(st) + 2, acc = w.stage_base(st);
        const J* let = find_stmt(body, [&](const J& x) {
          const J* l = x.get("Let");
          return l && l->get("local") && l->get("local")->is_int && l->get("local")->i == (int64_t)val;
        });
        if (!let) {
          ok = false;
          break;
        }
        J init = *let->get("Let")->get("init");
        if (w.dtype != UNP_F64) {
          const J* c = init.get("Cast");
          if (!c || c->t != J::Arr || c->a.size() != 2) {
            ok = false;
            break;
          }
          J operand = c->a[0];  // copied out before `init` (which owns it) is replaced
          init = std::move(operand);
        }
        J pre;
        if (!unbind(w, init, st, pre)) {
          ok = false;
          break;
        }
        sp.pres.push_back(pre);
        const J* asg = find_stmt(body, [&](const J& x) {
          const J* a = x.get("Assign");
          return a && a->get("local") && a->get("local")->is_int && a->get("local")->i == (int64_t)acc;
        });
        const J* value = asg ? asg->get("Assign")->get("value") : nullptr;
        if (value && value->get("Add")) cand.push_back({UNP_OP_SUM, UNP_OP_MEAN});
        else if (value && value->get("Mul")) cand.push_back({UNP_OP_PROD});
        else cand.push_back({UNP_OP_MAX, UNP_OP_MIN});
      }
      const J* store = ok ? find_stmt(body, [&](const J& x) {
        const J* st = x.get("Store");
        const J* pl = st ? st->get("place") : nullptr;
        const J* lg = pl ? pl->get("Logical") : nullptr;
        return lg && lg->get("buffer") && lg->get("buffer")->is_int && lg->get("buffer")->i == (int64_t)n;
      })
                          : nullptr;
      if (!store || !unbind(w, *store->get("Store")->get("value"), S, sp.epilogue)) return false;
      // every combination of the candidate folds
      std::vector<size_t> pick(S, 0);
      for (;;) {
        sp.ops.clear();
        for (uint32_t st = 0; st < S; ++st) sp.ops.push_back(cand[st][pick[st]]);
        if (attempt([&] { return lift_row_reduce(name, sp, block, grid); })) return true;
        uint32_t st = 0;
        while (st < S && ++pick[st] == cand[st].size()) pick[st++] = 0;
        if (st == S) break;
      }
      return false;
    };
    bool found = try_row_reduce(k);
    // A kernel whose locals are numbered otherwise: renumbered into the numbering of each
    // candidate skeleton (the lift of every fold combination with Input(0) pres and epilogue;
    // at most 625 combinations, i.e. up to four stages).
    uint32_t combos = 1;
    for (uint32_t st = 0; st < S; ++st) combos *= 5;
    if (!found && S <= 4) {
      static const int32_t rops[] = {UNP_OP_SUM, UNP_OP_PROD, UNP_OP_MAX, UNP_OP_MIN, UNP_OP_MEAN};
      for (uint32_t c = 0; !found && c < combos; ++c) {
        RowReduceSpec proto_sp = sp;
        proto_sp.ops.clear();
        proto_sp.pres.assign(S, input_leaf(0));
        proto_sp.epilogue = input_leaf(0);
        for (uint32_t st = 0, q = c; st < S; ++st, q /= 5) proto_sp.ops.push_back(rops[q % 5]);
        J proto, kr;
        try {
          proto = lift_row_reduce(name, proto_sp, block, grid);
        } catch (const Decline&) {
          continue;
        }
        if (into_numbering_of(proto, kc, kr)) found = try_row_reduce(kr);
      }
    }
    if (found) {
      out.form.kind = UNP_FORM_ROW_REDUCE;
      out.form.dtype = sp.dtype;
      out.form.rank = sp.rank;
      out.rr = sp;
      out.lift = block ? "lift_row_reduce_opdef_launched" : "lift_row_reduce_opdef";
      return UNP_OK;
    }
  }
  why = "kernel `" + name +
        "` is not one of the forms this backend lowers (a lifted elementwise op, reduction, scan, row reduction or "
        "gather, the fused row fold, or the int4 dequant)";
  return UNP_UNSUPPORTED_KERNEL;
}

namespace {

int32_t emit(J k, char** json, unp_error* err) {
  const std::string s = kir::write(k);
  *json = static_cast<char*>(std::malloc(s.size() + 1));
  if (!*json) {
    set_error(err, UNP_INVALID_ARGUMENT, "out of memory");
    return UNP_INVALID_ARGUMENT;
  }
  std::memcpy(*json, s.c_str(), s.size() + 1);
  set_error(err, UNP_OK, "");
  return UNP_OK;
}

template <class F> int32_t lift_call(char** json, unp_error* err, F&& f) {
  if (!json) {
    set_error(err, UNP_INVALID_ARGUMENT, "null output");
    return UNP_INVALID_ARGUMENT;
  }
  *json = nullptr;
  try {
    return emit(f(), json, err);
  } catch (const Decline& d) {
    set_error(err, UNP_LIFT_DECLINE, d.what);
    return UNP_LIFT_DECLINE;
  }
}

}  // namespace
}  // namespace unp

extern "C" {

int32_t unp_lift_reduction(const char* name, int32_t dtype, int32_t rank, int32_t op, uint32_t axes_mask,
                           int32_t keepdim, uint32_t block, uint32_t grid, char** json, unp_error* err) {
  return unp::lift_call(json, err, [&] {
    return unp::lift_reduction(name ? name : "reduce", dtype, rank, op, axes_mask, keepdim != 0, block, grid);
  });
}

int32_t unp_lift_reduction_x(const char* name, int32_t dtype, int32_t rank, int32_t op, uint32_t axes_mask,
                             int32_t keepdim, int32_t n_inputs, const char* body_json, const char* post_json,
                             uint32_t block, uint32_t grid, char** json, unp_error* err) {
  using unp::kir::J;
  J body, post;
  std::string why;
  if (n_inputs < 1 || n_inputs > 8) {
    unp::set_error(err, UNP_INVALID_ARGUMENT, "a reduction reads 1 to 8 inputs");
    return UNP_INVALID_ARGUMENT;
  }
  if (!body_json || !unp::kir::parse(body_json, body, why)) {
    unp::set_error(err, UNP_PARSE_ERROR, "body: a ScalarExpr expected " + why);
    return UNP_PARSE_ERROR;
  }
  if (post_json && !unp::kir::parse(post_json, post, why)) {
    unp::set_error(err, UNP_PARSE_ERROR, "post: a ScalarExpr expected " + why);
    return UNP_PARSE_ERROR;
  }
  return unp::lift_call(json, err, [&] {
    return unp::lift_reduction(name ? name : "reduce", dtype, rank, op, axes_mask, keepdim != 0, block, grid,
                               (uint32_t)n_inputs, &body, post_json ? &post : nullptr);
  });
}

int32_t unp_lift_scan(const char* name, int32_t dtype, int32_t rank, int32_t op, int32_t axis, int32_t exclusive,
                      int32_t reverse, uint32_t block, uint32_t grid, char** json, unp_error* err) {
  return unp::lift_call(json, err, [&] {
    return unp::lift_scan(name ? name : "scan", dtype, rank, op, axis, exclusive != 0, reverse != 0, block, grid);
  });
}

int32_t unp_lift_scan_x(const char* name, int32_t dtype, int32_t rank, int32_t op, int32_t axis, int32_t exclusive,
                        int32_t reverse, int32_t n_inputs, const char* pre_json, const char* post_json, uint32_t block,
                        uint32_t grid, char** json, unp_error* err) {
  using unp::kir::J;
  J pre, post;
  std::string why;
  if (n_inputs < 1 || n_inputs > 8) {
    unp::set_error(err, UNP_INVALID_ARGUMENT, "a scan reads 1 to 8 inputs");
    return UNP_INVALID_ARGUMENT;
  }
  if (!pre_json || !unp::kir::parse(pre_json, pre, why)) {
    unp::set_error(err, UNP_PARSE_ERROR, "pre: a ScalarExpr expected " + why);
    return UNP_PARSE_ERROR;
  }
  if (post_json && !unp::kir::parse(post_json, post, why)) {
    unp::set_error(err, UNP_PARSE_ERROR, "post: a ScalarExpr expected " + why);
    return UNP_PARSE_ERROR;
  }
  return unp::lift_call(json, err, [&] {
    return unp::lift_scan(name ? name : "scan", dtype, rank, op, axis, exclusive != 0, reverse != 0, block, grid,
                          (uint32_t)n_inputs, &pre, post_json ? &post : nullptr);
  });
}

int32_t unp_lift_gather(const char* name, int32_t dtype, int32_t rank, int32_t index_dtype, int32_t axis,
                        int32_t oob, uint32_t block, uint32_t grid, char** json, unp_error* err) {
  return unp::lift_call(json, err, [&] {
    return unp::lift_gather(name ? name : "gather", dtype, rank, index_dtype, axis, oob, block, grid);
  });
}

int32_t unp_lift_gather_x(const char* name, int32_t dtype, int32_t rank, int32_t index_dtype, int32_t axis,
                          int32_t oob, int32_t n_inputs, int32_t data_slot, int32_t index_slot, const char* body_json,
                          uint32_t block, uint32_t grid, char** json, unp_error* err) {
  using unp::kir::J;
  J body;
  std::string why;
  if (!body_json || !unp::kir::parse(body_json, body, why)) {
    unp::set_error(err, UNP_PARSE_ERROR, "body: a ScalarExpr expected " + why);
    return UNP_PARSE_ERROR;
  }
  if (n_inputs < 2 || n_inputs > 8 || data_slot < 0 || index_slot < 0) {
    unp::set_error(err, UNP_LIFT_DECLINE, "UnsupportedForm: an ill-formed gather");
    return UNP_LIFT_DECLINE;
  }
  return unp::lift_call(json, err, [&] {
    return unp::lift_gather(name ? name : "gather", dtype, rank, index_dtype, axis, oob, block, grid,
                            (uint32_t)n_inputs, (uint32_t)data_slot, (uint32_t)index_slot, &body);
  });
}

int32_t unp_lift_elementwise(const char* name, int32_t dtype, int32_t rank, int32_t n_inputs, const char* body_json,
                             const int32_t* perms, uint32_t block, uint32_t grid, char** json, unp_error* err) {
  using unp::kir::J;
  J body;
  std::string why;
  if (!body_json || !unp::kir::parse(body_json, body, why)) {
    unp::set_error(err, UNP_PARSE_ERROR, "body: a ScalarExpr expected " + why);
    return UNP_PARSE_ERROR;
  }
  if (n_inputs < 1 || n_inputs > 8 || rank < 0 || rank > 8) {
    unp::set_error(err, UNP_LIFT_DECLINE, "UnsupportedForm: an elementwise op of 1 to 8 inputs at rank 1 to 8");
    return UNP_LIFT_DECLINE;
  }
  std::vector<std::vector<int32_t>> pm;
  if (perms)
    for (int32_t k = 0; k < n_inputs; ++k) pm.emplace_back(perms + (size_t)k * (size_t)rank, perms + (size_t)(k + 1) * (size_t)rank);
  return unp::lift_call(json, err, [&] {
    return unp::lift_elementwise(name ? name : "elementwise", dtype, rank, (uint32_t)n_inputs, body, pm, block, grid);
  });
}

int32_t unp_kernel_row_reduce2(const char* name, int32_t dtype, int32_t op0, int32_t op1, uint32_t block,
                               uint32_t grid, char** json, unp_error* err) {
  return unp::lift_call(json, err, [&] { return unp::row_reduce2(name ? name : "row_reduce2", dtype, op0, op1, block, grid); });
}

int32_t unp_kernel_dequant4(const char* name, int32_t q_kind, int32_t z_kind, int32_t group, uint32_t block,
                            uint32_t grid, char** json, unp_error* err) {
  return unp::lift_call(json, err, [&] { return unp::dequant4(name ? name : "dequant4", q_kind, z_kind, group, block, grid); });
}

int32_t unp_kernel_dequant_gemm(const char* name, int32_t w_kind, int32_t x_kind, int32_t group, uint32_t block,
                                uint32_t grid, char** json, unp_error* err) {
  return unp::lift_call(json, err, [&] {
    return unp::dequant_gemm(name ? name : "dequant_gemm", w_kind, x_kind, group, block, grid);
  });
}

int32_t unp_lift_row_reduce(const char* name, int32_t dtype, int32_t rank, int32_t n_inputs, const char* stages_json,
                            const char* epilogue_json, uint32_t block, uint32_t grid, char** json, unp_error* err) {
  using unp::kir::J;
  unp::RowReduceSpec sp;
  sp.dtype = dtype;
  sp.rank = rank;
  sp.n_inputs = n_inputs;
  J stages, epi;
  std::string why;
  if (!stages_json || !unp::kir::parse(stages_json, stages, why) || stages.t != J::Arr) {
    unp::set_error(err, UNP_PARSE_ERROR, "stages: a JSON array of ReduceStage {pre, op} expected " + why);
    return UNP_PARSE_ERROR;
  }
  if (!epilogue_json || !unp::kir::parse(epilogue_json, epi, why)) {
    unp::set_error(err, UNP_PARSE_ERROR, "epilogue: a ScalarExpr expected " + why);
    return UNP_PARSE_ERROR;
  }
  for (const J& st : stages.a) {
    const J* pre = st.get("pre");
    const J* op = st.get("op");
    if (!pre || !op || op->t != J::Str) {
      unp::set_error(err, UNP_PARSE_ERROR, "a ReduceStage is {\"pre\": ScalarExpr, \"op\": ReduceOp}");
      return UNP_PARSE_ERROR;
    }
    int32_t code = -1;
    static const char* const names[] = {"Sum", "Prod", "Max", "Min", "Mean"};
    for (int32_t i = 0; i < 5; ++i)
      if (op->s == names[i]) code = i;
    sp.ops.push_back(code);
    sp.pres.push_back(*pre);
  }
  sp.epilogue = epi;
  return unp::lift_call(json, err, [&] { return unp::lift_row_reduce(name ? name : "row_reduce", sp, block, grid); });
}

}  // extern "C"
