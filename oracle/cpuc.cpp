// The reference's portable-C99 CPU leg, restated -- TEST INFRASTRUCTURE ONLY.
//
// EvansLaboratories/Unpopped ships one in-tree emitter, `unpopped-cpu-c`, that lowers a kernel-layer
// `KernelFn` to C99 (crates/unpopped-cpu-c/src/lib.rs:163 -> kernel.rs:598).  It is the second
// parity reference and the CPU baseline for the HIP backend's hot path.  The reference is Rust and
// cannot be built here, so this file restates its scheme in C++ over the serde JSON form of a
// KernelFn:
//
//  * the C function `int unpopped_cpu_kernel_<name>(...)` returns 0 when the kernel finished, 1 when
//    an access fell outside its buffer and 2 for a zero loop step (kernel.rs:9-11; 3, a bad grid,
//    belongs to grids read from arguments, which this restatement refuses);
//  * a buffer parameter i is four C arguments `T* bI, const long long* bI_shape,
//    const long long* bI_stride, long long bI_base` (`const T*` unless written), a scalar is `T pI`
//    (base.rs:65-103);
//  * every buffer and allocation access is bounds-checked per coordinate (kernel.rs:540-553,
//    launch.rs alloc_address); a sub-byte load unpacks the nibble, low nibble first, sign-extending
//    an I4 (kernel.rs:515-536);
//  * a launched kernel is a serialized thread loop: blocks ascend, threads ascend, each thread runs to
//    the next barrier before the next starts, locals become per-thread arrays and a construct that
//    holds a barrier is block level, read at thread 0 (launch.rs:1-45, 277-640);
//  * expressions follow the reference's C spellings: integer + - * wrap through the unsigned type,
//    integer / and shifts go through total helpers (typed.rs:27-76, 326-499); casts round to nearest
//    even or decline, float-to-integer saturates with NaN to 0 (typed.rs:113-216); F32 arithmetic is
//    C's per-operation float arithmetic, comparisons at F32 compute are decided on (float) operands,
//    Max/Min propagate NaN and pick the first operand on ties (cfamily.rs:886-1082); F16/Bf16 are
//    16-bit patterns that only a Cast decodes or encodes, through an emitted software codec that
//    rounds once to nearest even (narrow.rs, cfamily.rs:223-304).
//
// The emitted text is this build's own; only the scheme, the ABI and the rounding rules follow the
// reference, because parity with its C leg is defined by them.  A kernel outside the subset is a
// typed refusal (LowerError::UnsupportedKernel), never an approximation.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace {

// ---- JSON ---------------------------------------------------------------------------------------
struct V {
  enum T { Null, Bool, Int, Dbl, Str, Arr, Obj } t = Null;
  bool b = false;
  long long i = 0;
  double d = 0.0;
  std::string s;
  std::vector<V> a;
  std::vector<std::pair<std::string, V>> o;
  const V* get(const char* k) const {
    if (t != Obj) return nullptr;
    for (const auto& kv : o)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct Reader {
  const char* p;
  const char* end;
  std::string err;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\t' || *p == '\r')) ++p;
  }
  bool fail(const char* m) {
    if (err.empty()) err = m;
    return false;
  }
  bool str(std::string& out) {
    if (p >= end || *p != '"') return fail("expected a string");
    ++p;
    while (p < end && *p != '"') {
      char c = *p++;
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (p >= end) return fail("bad escape");
      char e = *p++;
      switch (e) {
        case 'n': out.push_back('\n'); break;
        case 't': out.push_back('\t'); break;
        case 'r': out.push_back('\r'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'u': {
          if (end - p < 4) return fail("bad \\u escape");
          unsigned cp = (unsigned)strtoul(std::string(p, 4).c_str(), nullptr, 16);
          p += 4;
          if (cp < 0x80) {
            out.push_back((char)cp);
          } else if (cp < 0x800) {
            out.push_back((char)(0xC0 | (cp >> 6)));
            out.push_back((char)(0x80 | (cp & 63)));
          } else {
            out.push_back((char)(0xE0 | (cp >> 12)));
            out.push_back((char)(0x80 | ((cp >> 6) & 63)));
            out.push_back((char)(0x80 | (cp & 63)));
          }
          break;
        }
        default: out.push_back(e);
      }
    }
    if (p >= end) return fail("unterminated string");
    ++p;
    return true;
  }
  bool val(V& v, int depth) {
    if (depth > 512) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    char c = *p;
    if (c == '{') {
      v.t = V::Obj;
      ++p;
      ws();
      if (p < end && *p == '}') {
        ++p;
        return true;
      }
      for (;;) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= end || *p != ':') return fail("expected ':'");
        ++p;
        V x;
        if (!val(x, depth + 1)) return false;
        v.o.emplace_back(std::move(k), std::move(x));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') {
          ++p;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.t = V::Arr;
      ++p;
      ws();
      if (p < end && *p == ']') {
        ++p;
        return true;
      }
      for (;;) {
        V x;
        if (!val(x, depth + 1)) return false;
        v.a.push_back(std::move(x));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') {
          ++p;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.t = V::Str;
      return str(v.s);
    }
    if (!strncmp(p, "true", 4)) {
      v.t = V::Bool;
      v.b = true;
      p += 4;
      return true;
    }
    if (!strncmp(p, "false", 5)) {
      v.t = V::Bool;
      p += 5;
      return true;
    }
    if (!strncmp(p, "null", 4)) {
      p += 4;
      return true;
    }
    const char* q = p;
    bool frac = false;
    if (q < end && (*q == '-' || *q == '+')) ++q;
    while (q < end && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' || *q == '-' || *q == '+')) {
      if (*q == '.' || *q == 'e' || *q == 'E') frac = true;
      ++q;
    }
    if (q == p) return fail("unexpected character");
    std::string num(p, q);
    p = q;
    if (frac) {
      v.t = V::Dbl;
      v.d = strtod(num.c_str(), nullptr);
    } else {
      v.t = V::Int;
      v.i = strtoll(num.c_str(), nullptr, 10);
      v.d = (double)v.i;
    }
    return true;
  }
};

// ---- refusals -----------------------------------------------------------------------------------
struct Refuse {
  std::string why;
};
[[noreturn]] void refuse(const std::string& why) { throw Refuse{why}; }

// An externally tagged serde enum value: its variant name and payload (nullptr for a unit variant).
std::string tag_of(const V& v, const V** payload) {
  *payload = nullptr;
  if (v.t == V::Str) return v.s;
  if (v.t == V::Obj && v.o.size() == 1) {
    *payload = &v.o[0].second;
    return v.o[0].first;
  }
  refuse("a malformed enum value");
}
const V& field(const V& v, const char* k) {
  const V* f = v.get(k);
  if (!f) refuse(std::string("missing field `") + k + "`");
  return *f;
}
long long as_int(const V& v) {
  if (v.t != V::Int) refuse("expected an integer");
  return v.i;
}
const std::string& as_str(const V& v) {
  if (v.t != V::Str) refuse("expected a string");
  return v.s;
}
const V& arr_at(const V& v, size_t i) {
  if (v.t != V::Arr || i >= v.a.size()) refuse("expected an array element");
  return v.a[i];
}

// ---- element kinds (crates/unpopped-vocab/src/element.rs:1052) ------------------------------------
bool is_narrow(const std::string& t) { return t == "F16" || t == "Bf16"; }
bool is_subbyte(const std::string& t) { return t == "I4" || t == "U4"; }
bool is_cast_float(const std::string& t) { return t == "F32" || t == "F32Strict" || t == "F64"; }
bool is_cast_int(const std::string& t) {
  return t == "I8" || t == "I16" || t == "I32" || t == "I64" || t == "U8" || t == "U16" || t == "U32" || t == "U64";
}
bool is_int_compute(const std::string& t) { return t == "I32" || t == "I64" || t == "U32" || t == "U64"; }
int int_bits(const std::string& t) {
  if (t == "I8" || t == "U8") return 8;
  if (t == "I16" || t == "U16") return 16;
  if (t == "I32" || t == "U32") return 32;
  return 64;
}
bool is_signed_int(const std::string& t) { return t[0] == 'I'; }

// The C type of a value in the typed table (typed.rs:79-94), or nullptr.
const char* c_type(const std::string& t) {
  if (t == "F32" || t == "F32Strict") return "float";
  if (t == "F64") return "double";
  if (t == "I8") return "signed char";
  if (t == "I16") return "short";
  if (t == "I32") return "int";
  if (t == "I64") return "long long";
  if (t == "U8") return "unsigned char";
  if (t == "U16") return "unsigned short";
  if (t == "U32") return "unsigned int";
  if (t == "U64") return "unsigned long long";
  return nullptr;
}
// The C type of a local or scalar (base.rs:19-32): a nibble lives widened, a half as its pattern.
const char* ctype(const std::string& t, const std::string& what) {
  if (t == "I4") return "signed char";
  if (t == "U4") return "unsigned char";
  if (is_narrow(t)) return "unsigned short";
  const char* c = c_type(t);
  if (!c) refuse(what + " has dtype " + t + ", which this emitter does not spell");
  return c;
}

std::string ll_lit(long long v) {
  if (v == INT64_MIN) return "(-9223372036854775807LL - 1)";
  return std::to_string(v) + "LL";
}
void int_range(const std::string& t, long long& lo, long long& hi) {
  int b = int_bits(t);
  if (is_signed_int(t)) {
    hi = b == 64 ? INT64_MAX : (1LL << (b - 1)) - 1;
    lo = b == 64 ? INT64_MIN : -(1LL << (b - 1));
  } else {
    lo = 0;
    hi = b == 64 ? INT64_MAX : (1LL << b) - 1;
  }
}
// Whether a conversion from -> to can be inexact.
bool rounding_matters(const std::string& from, const std::string& to) {
  if (from == to) return false;
  const bool ff = is_cast_float(from) || is_narrow(from), tf = is_cast_float(to) || is_narrow(to);
  auto mant = [](const std::string& t) { return t == "F64" ? 53 : t == "F16" ? 11 : t == "Bf16" ? 8 : 24; };
  if (ff && tf) return mant(to) < mant(from) || is_narrow(to);
  if (ff && !tf) return true;
  if (!ff && tf) return int_bits(from) - (is_signed_int(from) ? 1 : 0) > mant(to);
  return false;
}

// A finite or special double as a C99 literal.
std::string const_lit(double v) {
  if (std::isnan(v)) return "NAN";
  if (std::isinf(v)) return v > 0 ? "INFINITY" : "(-INFINITY)";
  char buf[64];
  snprintf(buf, sizeof buf, "%.17g", v);
  std::string s = buf;
  if (s.find_first_of(".eE") == std::string::npos) s += ".0";
  if (v < 0 || (v == 0 && std::signbit(v))) s = "(" + s + ")";
  return s;
}
double const_value(const V& p) {
  if (p.t == V::Str) {
    if (p.s == "NaN") return NAN;
    if (p.s == "inf") return INFINITY;
    if (p.s == "-inf") return -INFINITY;
    refuse("a Const that is not a number");
  }
  if (p.t != V::Int && p.t != V::Dbl) refuse("a Const that is not a number");
  return p.d;
}

// ---- the kernel ---------------------------------------------------------------------------------
struct Param {
  std::string name;
  bool buffer = false;
  std::string elem, role;  // buffer
  std::string ty;          // scalar
  long long local = -1;    // scalar
};
struct Alloc {
  std::string name, space, elem;
  long long extent = 0;
};
struct Launch {
  long long block[3] = {1, 1, 1}, grid[3] = {1, 1, 1};
  long long threads() const { return block[0] * block[1] * block[2]; }
};

struct Kernel {
  std::string name, compute;
  std::vector<Param> params;
  std::vector<std::string> locals;
  const V* body = nullptr;
  bool launched = false;
  Launch launch;
  std::vector<Alloc> allocs;
};

constexpr long long kMaxThreads = 1024;  // launch.rs:55-56: per-thread local arrays live on the stack

Kernel read_kernel(const V& k) {
  Kernel K;
  K.name = as_str(field(k, "name"));
  K.compute = as_str(field(k, "compute"));
  for (const V& p : field(k, "params").a) {
    Param P;
    P.name = as_str(field(p, "name"));
    const V* pay;
    const std::string kind = tag_of(field(p, "kind"), &pay);
    if (kind == "Buffer" && pay) {
      P.buffer = true;
      P.elem = as_str(field(*pay, "elem"));
      P.role = as_str(field(*pay, "role"));
    } else if (kind == "Scalar" && pay) {
      P.ty = as_str(field(*pay, "ty"));
      P.local = as_int(field(*pay, "local"));
    } else {
      refuse("a parameter kind this emitter has not been taught (" + kind + ")");
    }
    K.params.push_back(P);
  }
  for (const V& l : field(k, "locals").a) {
    const V* lanes = l.get("lanes");
    if (lanes && lanes->t == V::Int && lanes->i != 1) refuse("a packed local");
    K.locals.push_back(as_str(field(l, "elem")));
  }
  K.body = &field(k, "body");
  if (K.body->t != V::Arr) refuse("the body is not a block");
  const V* L = k.get("launch");
  if (L && L->t == V::Obj) {
    K.launched = true;
    for (int a = 0; a < 3; ++a) {
      K.launch.block[a] = as_int(arr_at(field(*L, "block"), a));
      K.launch.grid[a] = as_int(arr_at(field(*L, "grid"), a));
    }
    const V* gd = L->get("grid_dims");
    if (gd && gd->t != V::Null) refuse("a grid read from scalar arguments");
    const V* dv = L->get("devices");
    if (dv && dv->t == V::Int && dv->i != 1) refuse("a launch of several devices");
    const V* cl = L->get("cluster");
    if (cl && cl->t != V::Null) refuse("a launch with clusters");
  }
  if (const V* al = k.get("allocs")) {
    for (const V& a : al->a) {
      Alloc A;
      A.name = as_str(field(a, "name"));
      const V* pay;
      A.space = tag_of(field(a, "space"), &pay);
      A.elem = as_str(field(a, "elem"));
      const std::string ext = tag_of(field(a, "extent"), &pay);
      if (ext != "Static" || !pay) refuse("allocation `" + A.name + "` has a dynamic extent");
      A.extent = as_int(*pay);
      K.allocs.push_back(A);
    }
  }
  if (const V* r = k.get("results"))
    if (r->t == V::Arr && !r->a.empty()) refuse("a kernel with results (a callee)");
  return K;
}

// Everything about the kernel the emitter cannot do, refused before any text is written
// (kernel.rs:41-97, launch.rs:63-113).
void admit(const Kernel& K) {
  static const char* computes[] = {"F32", "F16", "Bf16", "F64", "I32", "I64", "U32", "U64"};
  bool ok = false;
  for (const char* c : computes) ok |= K.compute == c;
  if (!ok) refuse("compute dtype " + K.compute + "; only F32, F16, Bf16, F64, I32, I64, U32 and U64");
  for (const Param& p : K.params) ctype(p.buffer ? p.elem : p.ty, (p.buffer ? "buffer `" : "scalar `") + p.name + "`");
  for (size_t i = 0; i < K.locals.size(); ++i) ctype(K.locals[i], "local " + std::to_string(i));
  if (!K.launched && !K.allocs.empty()) refuse("an allocation without a launch shape");
  if (K.launched) {
    const long long nt = K.launch.threads();
    if (nt < 1 || nt > kMaxThreads) refuse("a block of " + std::to_string(nt) + " threads (1 to 1024 are spelled)");
    for (const Alloc& a : K.allocs) {
      if (a.space != "Shared" && a.space != "Private") refuse("allocation `" + a.name + "` is " + a.space);
      ctype(a.elem, "allocation `" + a.name + "`");
    }
  }
}

// ---- expressions --------------------------------------------------------------------------------
// The tree the spellers walk: an owned copy, so the narrow-float rewrites can build new nodes.
struct E {
  std::string tag;          // variant name
  std::string op;           // Binary/Unary op, Exec id, Cast/Bitcast target, ConstInt kind
  std::string round, sat;   // Cast
  double num = 0;           // Const
  long long ival = 0;       // ConstInt value, Local id, Exec axis
  std::vector<E> kids;
};

E read_expr(const V& v) {
  const V* p;
  E e;
  e.tag = tag_of(v, &p);
  const std::string& t = e.tag;
  if (t == "Const") {
    if (!p) refuse("Const without a value");
    e.num = const_value(*p);
  } else if (t == "ConstInt") {
    e.ival = as_int(arr_at(*p, 0));
    e.op = as_str(arr_at(*p, 1));
  } else if (t == "Local") {
    e.ival = as_int(*p);
  } else if (t == "Exec") {
    const V* ap;
    e.op = tag_of(*p, &ap);
    e.ival = ap ? as_int(*ap) : -1;
  } else if (t == "Add" || t == "Sub" || t == "Mul" || t == "Div") {
    e.kids = {read_expr(arr_at(*p, 0)), read_expr(arr_at(*p, 1))};
  } else if (t == "Binary") {
    e.op = as_str(arr_at(*p, 0));
    e.kids = {read_expr(arr_at(*p, 1)), read_expr(arr_at(*p, 2))};
  } else if (t == "Unary") {
    e.op = as_str(arr_at(*p, 0));
    e.kids = {read_expr(arr_at(*p, 1))};
  } else if (t == "Select" || t == "Fma") {
    e.kids = {read_expr(arr_at(*p, 0)), read_expr(arr_at(*p, 1)), read_expr(arr_at(*p, 2))};
  } else if (t == "Cast") {
    e.kids = {read_expr(arr_at(*p, 0))};
    const V& spec = arr_at(*p, 1);
    e.op = as_str(field(spec, "to"));
    const V* r = spec.get("round");
    const V* s = spec.get("sat");
    e.round = r ? as_str(*r) : "NearestEven";
    e.sat = s ? as_str(*s) : "Wrap";
  } else if (t == "Bitcast") {
    e.kids = {read_expr(arr_at(*p, 0))};
    e.op = as_str(arr_at(*p, 1));
  } else if (t == "Input" || t == "Param" || t == "Reduced" || t == "Coord" || t == "CoordInt") {
    refuse("an " + t + " leaf inside a kernel; the checker rejects it");
  } else {
    refuse("the expression node " + t + ", which this emitter does not spell");
  }
  return e;
}

E cast_node(E x, const std::string& to) {
  E c;
  c.tag = "Cast";
  c.op = to;
  c.round = "NearestEven";
  c.sat = "Wrap";
  c.kids.push_back(std::move(x));
  return c;
}

bool is_cmp(const std::string& op) {
  return op == "CmpEq" || op == "CmpNe" || op == "CmpLt" || op == "CmpLe" || op == "CmpGt" || op == "CmpGe";
}

struct Emitter {
  const Kernel& K;
  std::string out;
  int depth = 1;
  unsigned fresh = 0;
  int thread_loops = 0;
  bool has_return = false;

  explicit Emitter(const Kernel& k) : K(k) {}

  void line(const std::string& s) {
    out.append(4 * depth, ' ');
    out += s;
    out += '\n';
  }

  // The dtype a float operator is spelled at: the compute dtype, a narrow one computed as F32.
  std::string math_dtype() const { return is_narrow(K.compute) ? "F32" : K.compute; }

  // ---- typing (crates/unpopped/src/types.rs, as far as the spellers need it) ----
  std::string ty(const E& e) const {
    const std::string& t = e.tag;
    if (t == "Const") return K.compute;
    if (t == "ConstInt") return e.op;
    if (t == "Local") {
      if (e.ival < 0 || (size_t)e.ival >= K.locals.size()) refuse("a Local that is not declared");
      return K.locals[(size_t)e.ival];
    }
    if (t == "Exec") return "U32";
    if (t == "Cast" || t == "Bitcast") return e.op;
    if (t == "Binary" && is_cmp(e.op)) return K.compute;
    if (t == "Select") return ty(e.kids[1]);
    return ty(e.kids[0]);
  }

  // ---- F16/Bf16: patterns that only a Cast decodes or encodes (narrow.rs) ----
  // The narrow float `e` is typed as, or "".
  std::string narrow_ty(const E& e) const {
    const std::string& t = e.tag;
    if (t == "Const") return is_narrow(K.compute) ? K.compute : "";
    if (t == "Local") {
      const std::string& l = K.locals.at((size_t)e.ival);
      return is_narrow(l) ? l : "";
    }
    if (t == "Cast") return is_narrow(e.op) ? e.op : "";
    if (t == "Bitcast" || t == "ConstInt" || t == "Exec") return "";
    if (t == "Select") {
      std::string a = narrow_ty(e.kids[1]);
      return a.empty() ? narrow_ty(e.kids[2]) : a;
    }
    for (const E& k : e.kids) {
      std::string n = narrow_ty(k);
      if (!n.empty()) return n;
    }
    return "";
  }
  static bool is_pattern(const E& e) { return e.tag == "Local" || e.tag == "Cast"; }
  // `e` as a value C computes on: every narrow operand decoded to float.
  E wide(const E& e) const {
    if (e.tag == "Cast") {
      E inner = e;
      inner.kids[0] = moved(e.kids[0]);
      return is_narrow(e.op) ? cast_node(inner, "F32") : inner;
    }
    if (!narrow_ty(e).empty() && is_pattern(e)) return cast_node(e, "F32");
    E r = e;
    const bool narrow_cmp = e.tag == "Binary" && is_cmp(e.op) && is_narrow(K.compute);
    for (size_t i = 0; i < r.kids.size(); ++i) {
      if (narrow_cmp && r.kids[i].tag == "Const")
        r.kids[i] = cast_node(cast_node(r.kids[i], K.compute), "F32");
      else
        r.kids[i] = wide(e.kids[i]);
    }
    return r;
  }
  // `e` as a value that is bound or stored: a bare pattern stays one, narrow arithmetic is computed
  // wide and encoded once.
  E moved(const E& e) const {
    if (e.tag == "Cast") {
      E r = e;
      r.kids[0] = moved(e.kids[0]);
      return r;
    }
    const std::string n = narrow_ty(e);
    if (!n.empty() && is_pattern(e)) return e;
    if (!n.empty() && e.tag == "Select") refuse("a Select between narrow-float patterns");
    if (!n.empty()) return cast_node(wide(e), n);
    return wide(e);
  }

  // ---- spellings ----
  std::string local_ref(long long l) const {
    return K.launched ? "l" + std::to_string(l) + "[t]" : "l" + std::to_string(l);
  }

  std::string exec_c(const E& e) const {
    if (!K.launched) refuse("an execution id without a launch shape");
    const long long a = e.ival;
    const Launch& L = K.launch;
    if (e.op == "ThreadIdx" && a == 0) return "((unsigned int)(t % " + std::to_string(L.block[0]) + "))";
    if (e.op == "ThreadIdx" && a == 1)
      return "((unsigned int)((t / " + std::to_string(L.block[0]) + ") % " + std::to_string(L.block[1]) + "))";
    if (e.op == "ThreadIdx" && a == 2) return "((unsigned int)(t / " + std::to_string(L.block[0] * L.block[1]) + "))";
    if (e.op == "BlockIdx" && a >= 0 && a <= 2) return "((unsigned int)blk" + std::to_string(a) + ")";
    if (e.op == "BlockDim" && a >= 0 && a <= 2) return std::to_string(L.block[a]) + "u";
    if (e.op == "GridDim" && a >= 0 && a <= 2) return std::to_string(L.grid[a]) + "u";
    refuse("the execution id " + e.op);
  }

  // An integer operation at type t (typed.rs cpu_int_op): + - * wrap through the unsigned type.
  std::string int_op(const std::string& op, const std::string& t, const std::vector<std::string>& x) const {
    const char* c = c_type(t);
    if (!c || !is_cast_int(t)) refuse("integer arithmetic at " + t);
    const std::string wide = int_bits(t) == 64 ? "unsigned long long" : "unsigned int";
    const std::string cs = c;
    if (op == "Add" || op == "Sub" || op == "Mul") {
      const char* sym = op == "Add" ? " + " : op == "Sub" ? " - " : " * ";
      return "((" + cs + ")((" + wide + ")(" + x[0] + ")" + sym + "(" + wide + ")(" + x[1] + ")))";
    }
    if (op == "Min" || op == "Max") {
      const char* sym = op == "Min" ? " < " : " > ";
      return "((" + cs + ")((" + x[0] + ")" + sym + "(" + x[1] + ") ? (" + x[0] + ") : (" + x[1] + ")))";
    }
    if (op == "Select") return "((" + cs + ")((" + x[0] + ") != 0 ? (" + x[1] + ") : (" + x[2] + ")))";
    if (is_cmp(op)) {
      const std::string& k = K.compute;
      const char* one = k == "F64" ? "1.0" : is_int_compute(k) ? "1" : "1.0f";
      const char* zero = k == "F64" ? "0.0" : is_int_compute(k) ? "0" : "0.0f";
      const char* sym = op == "CmpEq" ? " == " : op == "CmpNe" ? " != " : op == "CmpLt" ? " < " : op == "CmpLe" ? " <= "
                        : op == "CmpGt" ? " > " : " >= ";
      return "((" + x[0] + ")" + sym + "(" + x[1] + ") ? " + one + " : " + zero + ")";
    }
    if (op == "BitAnd") return "(" + x[0] + " & " + x[1] + ")";
    if (op == "BitOr") return "(" + x[0] + " | " + x[1] + ")";
    if (op == "BitXor") return "(" + x[0] + " ^ " + x[1] + ")";
    if (op == "Div" || op == "Shl" || op == "Shr") {
      if (!is_int_compute(t)) refuse("an integer " + op + " at " + t);
      std::string tt = t;
      for (char& ch : tt) ch = (char)tolower(ch);
      const std::string name = op == "Div" ? "div" : op == "Shl" ? "shl" : "shr";
      return "leg_" + name + "_" + tt + "(" + x[0] + ", " + x[1] + ")";
    }
    refuse("the integer operation " + op);
  }

  std::string unary(const std::string& op, const std::string& x) const {
    const std::string d = math_dtype();
    if (d != "F32" && d != "F32Strict" && d != "F64") refuse("the Unary " + op + " at compute " + K.compute);
    const bool f = d != "F64";
    const std::string one = f ? "1.0f" : "1.0", zero = f ? "0.0f" : "0.0", s = f ? "f" : "";
    if (op == "Neg") return "(-" + x + ")";
    if (op == "Abs") return "fabs" + s + "(" + x + ")";
    if (op == "Sqr") return "(" + x + "*" + x + ")";
    if (op == "Rsqrt") return "(" + one + "/sqrt" + s + "(" + x + "))";
    if (op == "Recip") return "(" + one + "/" + x + ")";
    if (op == "Sigmoid") return "(" + one + "/(" + one + "+exp" + s + "(-" + x + ")))";
    if (op == "Relu") return "(" + x + " < " + zero + " ? " + zero + " : " + x + ")";
    if (op == "Gelu")
      return "(" + std::string(f ? "0.5f" : "0.5") + "*" + x + "*(" + one + "+erf" + s + "(" + x + "*" +
             (f ? "0.70710678f" : "0.7071067811865476") + ")))";
    if (op == "Silu") return "(" + x + "*(" + one + "/(" + one + "+exp" + s + "(-" + x + "))))";
    if (op == "Sign") return "(" + x + " > " + zero + " ? " + one + " : (" + x + " < " + zero + " ? -" + one + " : " + zero + "))";
    if (op == "Step") return "(" + x + " > " + zero + " ? " + one + " : " + zero + ")";
    if (op == "Round") return "rint" + s + "(" + x + ")";
    static const char* const fns[][2] = {
        {"Sqrt", "sqrt"}, {"Exp", "exp"},     {"Log", "log"},     {"Tanh", "tanh"},   {"Erf", "erf"},
        {"Sin", "sin"},   {"Cos", "cos"},     {"Floor", "floor"}, {"Ceil", "ceil"},   {"Erfc", "erfc"},
        {"Trunc", "trunc"}, {"Exp2", "exp2"}, {"Expm1", "expm1"}, {"Log2", "log2"},   {"Log10", "log10"},
        {"Log1p", "log1p"}, {"Sinh", "sinh"}, {"Cosh", "cosh"},   {"Tan", "tan"},     {"Asin", "asin"},
        {"Acos", "acos"}, {"Atan", "atan"},   {"Asinh", "asinh"}, {"Acosh", "acosh"}, {"Atanh", "atanh"},
        {"Cbrt", "cbrt"}, {"Lgamma", "lgamma"}};
    for (const auto& fn : fns)
      if (op == fn[0]) return std::string(fn[1]) + s + "(" + x + ")";
    refuse("the Unary " + op);
  }

  std::string binary_float(const std::string& op, const std::string& a, const std::string& b) const {
    const std::string d = math_dtype();
    if (d != "F32" && d != "F32Strict" && d != "F64") refuse("the float Binary " + op + " at compute " + K.compute);
    const bool f = d != "F64";
    const std::string s = f ? "f" : "";
    if (op == "Max") return "(" + a + " != " + a + " ? " + a + " : (" + b + " != " + b + " ? " + b + " : (" + a + " >= " + b + " ? " + a + " : " + b + ")))";
    if (op == "Min") return "(" + a + " != " + a + " ? " + a + " : (" + b + " != " + b + " ? " + b + " : (" + a + " <= " + b + " ? " + a + " : " + b + ")))";
    if (op == "Pow") return "pow" + s + "(" + a + ", " + b + ")";
    if (op == "Rem") return "(" + a + " - floor" + s + "(" + a + " / " + b + ") * " + b + ")";
    if (op == "Atan2") return "atan2" + s + "(" + a + ", " + b + ")";
    if (op == "Copysign") return "copysign" + s + "(" + a + ", " + b + ")";
    if (op == "Nextafter") return "nextafter" + s + "(" + a + ", " + b + ")";
    if (op == "FmaxIeee") return "fmax" + s + "(" + a + ", " + b + ")";
    if (op == "FminIeee") return "fmin" + s + "(" + a + ", " + b + ")";
    if (op == "RemTrunc") return "fmod" + s + "(" + a + ", " + b + ")";
    if (is_cmp(op)) {
      const char* sym = op == "CmpEq" ? " == " : op == "CmpNe" ? " != " : op == "CmpLt" ? " < " : op == "CmpLe" ? " <= "
                        : op == "CmpGt" ? " > " : " >= ";
      if (f) return "((float)" + a + sym + "(float)" + b + " ? 1.0f : 0.0f)";
      return "(" + a + sym + b + " ? 1.0 : 0.0)";
    }
    refuse("the Binary " + op + " on float operands");
  }

  std::string sub_byte_cast(const std::string& x, const std::string& from, const std::string& to) const {
    if (to == "I4") return "((signed char)(((((long long)(" + x + ")) + 8) & 15) - 8))";
    if (to == "U4") return "((unsigned char)(((long long)(" + x + ")) & 15))";
    const char* c = c_type(to);
    if (c && is_cast_int(to)) return "((" + std::string(c) + ")(" + x + "))";
    refuse("the Cast " + from + " -> " + to);
  }

  std::string narrow_cast(const std::string& x, const std::string& from, const E& spec) const {
    const std::string& to = spec.op;
    if (is_narrow(to)) {
      if (spec.sat != "Wrap") refuse("a Cast to " + to + " with saturation " + spec.sat);
      if (rounding_matters(from, to) && spec.round != "NearestEven") refuse("a Cast to " + to + " rounding " + spec.round);
      // every source value is exact in a double, which the encoder rounds once
      const std::string enc = to == "F16" ? "leg_to_f16" : "leg_to_bf16";
      if (is_narrow(from)) return enc + "((double)" + std::string(from == "F16" ? "leg_f16_value" : "leg_bf16_value") + "(" + x + "))";
      if (from == "F32" || from == "F32Strict" || from == "I8" || from == "I16" || from == "U8" || from == "U16" ||
          from == "F64" || from == "I32" || from == "U32" || from == "I64" || from == "U64")
        return enc + "((double)(" + x + "))";
      refuse("the Cast " + from + " -> " + to);
    }
    const std::string dec = from == "F16" ? "leg_f16_value" : "leg_bf16_value";
    return cast(dec + "(" + x + ")", "F32", spec);
  }

  // Cast `x` of type `from` per `spec` (typed.rs:113-216).
  std::string cast(const std::string& x, const std::string& from, const E& spec) const {
    const std::string& to = spec.op;
    if (is_subbyte(from) || is_subbyte(to)) return sub_byte_cast(x, from, to);
    if (is_narrow(from) || is_narrow(to)) return narrow_cast(x, from, spec);
    if (from == "U64" || to == "U64") refuse("the u64 Cast " + from + " -> " + to);
    const char* fc = c_type(from);
    const char* tc = c_type(to);
    if (!fc || !tc) refuse("no C type for the Cast " + from + " -> " + to);
    const std::string t = tc;
    const bool ff = is_cast_float(from), tf = is_cast_float(to);
    if (rounding_matters(from, to) && !(ff && !tf) && spec.round != "NearestEven")
      refuse("an inexact " + from + " -> " + to + " Cast rounding " + spec.round);
    if (ff && tf) {
      if (spec.sat == "ClampFinite" && from == "F64" && to != from) {
        const std::string m = "3.4028234663852886e+38";
        return "((" + t + ")((" + x + ") != (" + x + ") ? (" + x + ") : ((" + x + ") > " + m + " ? " + m + " : ((" + x +
               ") < -" + m + " ? -" + m + " : (" + x + ")))))";
      }
      return "((" + t + ")(" + x + "))";
    }
    if (ff && !tf) {
      const std::string& r = spec.round;
      const char* rnd = r == "TowardZero" ? "trunc" : r == "NearestEven" ? "nearbyint" : r == "TowardNegInf" ? "floor"
                        : r == "TowardPosInf" ? "ceil" : r == "NearestAway" ? "round" : nullptr;
      if (!rnd) refuse("the rounding mode " + r);
      long long lo, hi;
      int_range(to, lo, hi);
      return "((" + t + ")leg_f2i_sat(" + rnd + "((double)(" + x + ")), " + ll_lit(lo) + ", " + ll_lit(hi) + "))";
    }
    if (!ff && tf) return "((" + t + ")(" + x + "))";
    if (spec.sat == "Clamp") {
      long long lo, hi;
      int_range(to, lo, hi);
      return "((" + t + ")leg_clamp((long long)(" + x + "), " + ll_lit(lo) + ", " + ll_lit(hi) + "))";
    }
    return "((" + t + ")(" + x + "))";
  }

  // The integer form of an Add/Sub/Mul/Binary/Select node, when its operands are integers (backend.rs
  // int_node): the operation and the type, or "" for a float node.
  std::string int_route(const E& e, std::string& op) const {
    size_t first = 0;
    if (e.tag == "Add" || e.tag == "Sub" || e.tag == "Mul" || e.tag == "Div") {
      op = e.tag;
    } else if (e.tag == "Binary") {
      op = e.op;
    } else if (e.tag == "Select") {
      op = "Select";
      first = 1;
    } else {
      return "";
    }
    std::string t;
    bool any_int = false, any_float = false;
    for (size_t i = first; i < e.kids.size(); ++i) {
      const std::string k = ty(e.kids[i]);
      if (is_subbyte(k)) refuse("arithmetic on a sub-byte value (the kernel widens it to an integer first)");
      if (is_cast_int(k)) {
        any_int = true;
        if (!t.empty() && t != k) refuse("an integer " + op + " over " + t + " and " + k);
        t = k;
      } else {
        any_float = true;
      }
    }
    if (any_int && any_float) refuse("a " + op + " over an integer and a float");
    return any_int ? t : "";
  }

  std::string spell(const E& e) const {
    std::string op;
    const std::string it = int_route(e, op);
    if (!it.empty()) {
      std::vector<std::string> x;
      for (const E& k : e.kids) x.push_back(spell(k));
      return int_op(op, it, x);
    }
    const std::string& t = e.tag;
    if (t == "Const") {
      const std::string lit = const_lit(e.num);
      return math_dtype() == "F32" ? "((float)" + lit + ")" : lit;
    }
    if (t == "ConstInt") {
      const char* c = c_type(e.op);
      if (!c || !is_cast_int(e.op)) refuse("an integer constant of type " + e.op);
      return "((" + std::string(c) + ")(" + ll_lit(e.ival) + "))";
    }
    if (t == "Local") return local_ref(e.ival);
    if (t == "Exec") return exec_c(e);
    if (t == "Add" || t == "Sub" || t == "Mul" || t == "Div") {
      if (is_int_compute(K.compute)) refuse("float arithmetic in an integer-compute kernel");
      const char* sym = t == "Add" ? " + " : t == "Sub" ? " - " : t == "Mul" ? " * " : " / ";
      return "(" + spell(e.kids[0]) + sym + spell(e.kids[1]) + ")";
    }
    if (t == "Binary") return binary_float(e.op, spell(e.kids[0]), spell(e.kids[1]));
    if (t == "Unary") return unary(e.op, spell(e.kids[0]));
    if (t == "Select") {
      const std::string d = math_dtype();
      const std::string c = spell(e.kids[0]), a = spell(e.kids[1]), b = spell(e.kids[2]);
      if (d == "F64") return "(((double)(" + c + ")) != 0.0 ? (double)(" + a + ") : (double)(" + b + "))";
      if (d == "F32" || d == "F32Strict") return "(((float)(" + c + ")) != 0.0f ? (float)(" + a + ") : (float)(" + b + "))";
      refuse("a float Select at compute " + K.compute);
    }
    if (t == "Fma") {
      const std::string d = K.compute;
      const std::string fn = d == "F64" ? "fma" : (d == "F32" || d == "F32Strict") ? "fmaf" : "";
      if (fn.empty()) refuse("an Fma at compute " + d);
      return fn + "(" + spell(e.kids[0]) + ", " + spell(e.kids[1]) + ", " + spell(e.kids[2]) + ")";
    }
    if (t == "Cast") return cast(spell(e.kids[0]), ty(e.kids[0]), e);
    if (t == "Bitcast") {
      const std::string from = ty(e.kids[0]);
      const char* fc = c_type(from);
      const char* tc = c_type(e.op);
      if (!fc || !tc) refuse("no C type for the Bitcast " + from + " -> " + e.op);
      return "((union { " + std::string(fc) + " a; " + tc + " b; }){ (" + spell(e.kids[0]) + ") }).b";
    }
    refuse("the expression node " + t);
  }

  std::string expr(const V& v) const { return spell(wide(read_expr(v))); }    // an operand
  std::string value(const V& v) const { return spell(moved(read_expr(v))); }  // a bound or stored value

  std::string local_ctype(long long l) const {
    if (l < 0 || (size_t)l >= K.locals.size()) refuse("a Local that is not declared");
    return ctype(K.locals[(size_t)l], "a local");
  }

  void bind_local(long long l, const std::string& v) {
    const std::string t = local_ctype(l);
    if (K.launched)
      line(local_ref(l) + " = (" + t + ")(" + v + ");");
    else
      line(t + " l" + std::to_string(l) + " = (" + t + ")(" + v + ");");
  }

  // ---- places ----
  const Param& buffer_param(long long b) const {
    if (b < 0 || (size_t)b >= K.params.size() || !K.params[(size_t)b].buffer) refuse("a place on a parameter that is not a buffer");
    return K.params[(size_t)b];
  }

  // An lvalue for the place, after the statements that bounds-check it; `nib` is set for a
  // sub-byte buffer, whose element is then read through the nibble unpack.
  std::string address(const V& place, std::string* nib) {
    const V* p;
    const std::string t = tag_of(place, &p);
    const unsigned n = fresh++;
    const std::string o = "o" + std::to_string(n);
    if (t == "Logical" && p) {
      const long long b = as_int(field(*p, "buffer"));
      const Param& P = buffer_param(b);
      const std::string bs = "b" + std::to_string(b);
      line("long long " + o + " = " + bs + "_base;");
      const V& coords = field(*p, "coords");
      for (size_t d = 0; d < coords.a.size(); ++d) {
        const std::string c = expr(coords.a[d]);
        const std::string ds = std::to_string(d);
        line("{ long long c = (long long)(" + c + "); if (c < 0 || c >= " + bs + "_shape[" + ds + "]) return 1; " + o +
             " += c * " + bs + "_stride[" + ds + "]; }");
      }
      if (is_subbyte(P.elem)) {
        if (!nib) refuse("a sub-byte buffer written (sub-byte stores are refused)");
        std::string x = "((" + bs + "[(" + o + ") >> 1] >> (((" + o + ") & 1) * 4)) & 15)";
        *nib = P.elem == "I4" ? "((" + x + " ^ 8) - 8)" : x;
      }
      return bs + "[" + o + "]";
    }
    if (t == "Alloc" && p) {
      if (!K.launched) refuse("a Place::Alloc without a launch shape");
      const long long a = as_int(field(*p, "alloc"));
      if (a < 0 || (size_t)a >= K.allocs.size()) refuse("a Place::Alloc of an undeclared allocation");
      const Alloc& A = K.allocs[(size_t)a];
      const std::string ext = std::to_string(A.extent);
      line("long long " + o + " = (long long)(" + expr(field(*p, "index")) + "); if (" + o + " < 0 || " + o + " >= " + ext +
           ") return 1;");
      if (A.space == "Private") return "sh" + std::to_string(a) + "[(long long)t * " + ext + " + " + o + "]";
      return "sh" + std::to_string(a) + "[" + o + "]";
    }
    refuse("the place " + t);
  }

  // ---- statements ----
  void block(const V& b) {
    if (b.t != V::Arr) refuse("a block that is not a statement list");
    for (const V& s : b.a) stmt(s);
  }
  void nested(const V& b) {
    ++depth;
    block(b);
    --depth;
  }

  void stmt(const V& s) {
    const V* p;
    const std::string t = tag_of(s, &p);
    if (t == "Let" || t == "Assign") {
      const long long l = as_int(field(*p, "local"));
      const std::string v = value(field(*p, t == "Let" ? "init" : "value"));
      if (t == "Let") {
        bind_local(l, v);
      } else {
        const std::string ct = local_ctype(l);
        line(local_ref(l) + " = (" + ct + ")(" + v + ");");
      }
    } else if (t == "Load") {
      const long long l = as_int(field(*p, "local"));
      std::string nib;
      std::string at = address(field(*p, "place"), &nib);
      bind_local(l, nib.empty() ? at : nib);
    } else if (t == "Store") {
      const std::string at = address(field(*p, "place"), nullptr);
      line(at + " = " + value(field(*p, "value")) + ";");
    } else if (t == "If") {
      line("if ((" + expr(field(*p, "cond")) + ") != 0) {");
      nested(field(*p, "then"));
      const V& els = field(*p, "els");
      if (els.t == V::Arr && !els.a.empty()) {
        line("} else {");
        nested(els);
      }
      line("}");
    } else if (t == "For") {
      const long long l = as_int(field(*p, "local"));
      const std::string ct = local_ctype(l);
      const std::string n = std::to_string(fresh++);
      const std::string st = expr(field(*p, "start")), en = expr(field(*p, "end")), sp = expr(field(*p, "step"));
      line("{");
      ++depth;
      line("long long s" + n + " = (long long)(" + st + "), e" + n + " = (long long)(" + en + "), t" + n + " = (long long)(" + sp + ");");
      line("if (t" + n + " == 0) return 2;");
      line("for (long long k" + n + " = s" + n + "; t" + n + " > 0 ? k" + n + " < e" + n + " : k" + n + " > e" + n + "; k" + n +
           " += t" + n + ") {");
      ++depth;
      bind_local(l, "k" + n);
      ++thread_loops;
      block(field(*p, "body"));
      --thread_loops;
      --depth;
      line("}");
      --depth;
      line("}");
    } else if (t == "While") {
      line("while ((" + expr(field(*p, "cond")) + ") != 0) {");
      ++thread_loops;
      nested(field(*p, "body"));
      --thread_loops;
      line("}");
    } else if (t == "Break" || t == "Continue") {
      if (K.launched && thread_loops == 0) refuse("a Break or Continue that leaves a loop holding a Barrier");
      line(t == "Break" ? "break;" : "continue;");
    } else if (t == "Return") {
      if (K.launched) {
        has_return = true;
        line("goto thread_end;");
      } else {
        line("return 0;");
      }
    } else if (t == "Fence") {
      // A fence orders nothing in a sequential program.
    } else if (t == "Barrier") {
      refuse(K.launched ? "a Barrier inside a thread run (a While, or a construct this emitter cannot split)"
                        : "a Barrier needs a launch");
    } else {
      refuse("the statement " + t);
    }
  }

  // ---- the serialized thread loop (launch.rs) ----
  static bool contains_barrier(const V& s) {
    const V* p;
    const std::string t = tag_of(s, &p);
    if (t == "Barrier") return true;
    if (t == "If" && p) return any_barrier(field(*p, "then")) || any_barrier(field(*p, "els"));
    if ((t == "For" || t == "While") && p) return any_barrier(field(*p, "body"));
    return false;
  }
  static bool any_barrier(const V& b) {
    if (b.t != V::Arr) return false;
    for (const V& s : b.a)
      if (contains_barrier(s)) return true;
    return false;
  }
  static bool any_return(const V& b) {
    if (b.t != V::Arr) return false;
    for (const V& s : b.a) {
      const V* p;
      const std::string t = tag_of(s, &p);
      if (t == "Return") return true;
      if (t == "If" && p && (any_return(field(*p, "then")) || any_return(field(*p, "els")))) return true;
      if ((t == "For" || t == "While") && p && any_return(field(*p, "body"))) return true;
    }
    return false;
  }
  // The statements a launched kernel may hold (launch.rs admit_stmts).
  static void admit_stmts(const V& b, bool barriers) {
    for (const V& s : b.a) {
      const V* p;
      const std::string t = tag_of(s, &p);
      if (t == "Barrier") {
        const V* pay;
        if (tag_of(field(*p, "scope"), &pay) != "Block") refuse("a Barrier of a scope other than Block");
        if (tag_of(field(*p, "kind"), &pay) != "Full") refuse("a named barrier");
      } else if (t == "Return" && barriers) {
        refuse("a Return in a kernel that has a Barrier");
      } else if (t == "While" && any_barrier(field(*p, "body"))) {
        refuse("a While loop that holds a Barrier");
      } else if (t == "If") {
        admit_stmts(field(*p, "then"), barriers);
        admit_stmts(field(*p, "els"), barriers);
      } else if (t == "For" || t == "While") {
        admit_stmts(field(*p, "body"), barriers);
      }
    }
  }

  void flush_run(std::vector<const V*>& run) {
    if (run.empty()) return;
    line("for (int t = 0; t < " + std::to_string(K.launch.threads()) + "; ++t) {");
    ++depth;
    thread_loops = 0;
    for (const V* s : run) stmt(*s);
    run.clear();
    --depth;
    if (any_return(*K.body)) line("thread_end: ;");
    line("}");
  }

  // A statement list at block level: each stretch of statements free of barriers is emitted as one
  // loop over the block's threads; a statement containing a barrier closes the stretch and is
  // emitted a single time, whatever condition or loop bounds it has evaluated as thread 0 sees them.
  void phases(const V& stmts) {
    std::vector<const V*> run;
    for (const V& s : stmts.a) {
      if (!contains_barrier(s)) {
        run.push_back(&s);
        continue;
      }
      flush_run(run);
      const V* p;
      const std::string t = tag_of(s, &p);
      if (t == "Barrier") {
        line("/* barrier: the thread loop ends here */");
      } else if (t == "If") {
        line("{");
        ++depth;
        line("const int t = 0;");
        line("if ((" + expr(field(*p, "cond")) + ") != 0) {");
        ++depth;
        phases(field(*p, "then"));
        --depth;
        line("} else {");
        ++depth;
        phases(field(*p, "els"));
        --depth;
        line("}");
        --depth;
        line("}");
      } else if (t == "For") {
        const long long l = as_int(field(*p, "local"));
        const std::string ct = local_ctype(l);
        const std::string n = std::to_string(fresh++);
        line("{");
        ++depth;
        line("const int t = 0;");
        line("long long s" + n + " = (long long)(" + expr(field(*p, "start")) + "), e" + n + " = (long long)(" +
             expr(field(*p, "end")) + "), t" + n + " = (long long)(" + expr(field(*p, "step")) + ");");
        line("if (t" + n + " == 0) return 2;");
        line("for (long long k" + n + " = s" + n + "; t" + n + " > 0 ? k" + n + " < e" + n + " : k" + n + " > e" + n + "; k" +
             n + " += t" + n + ") {");
        ++depth;
        line("for (int tt = 0; tt < " + std::to_string(K.launch.threads()) + "; ++tt) l" + std::to_string(l) + "[tt] = (" +
             ct + ")k" + n + ";");
        phases(field(*p, "body"));
        --depth;
        line("}");
        --depth;
        line("}");
      } else {
        refuse("a statement holding a Barrier this emitter cannot split");
      }
    }
    flush_run(run);
  }

  void launched_body() {
    admit_stmts(*K.body, any_barrier(*K.body));
    const std::string nt = std::to_string(K.launch.threads());
    for (size_t i = 0; i < K.locals.size(); ++i)
      line(std::string(ctype(K.locals[i], "a local")) + " l" + std::to_string(i) + "[" + nt + "];");
    for (size_t i = 0; i < K.params.size(); ++i) {
      const Param& P = K.params[i];
      if (!P.buffer)
        line("for (int t = 0; t < " + nt + "; ++t) l" + std::to_string(P.local) + "[t] = (" + ctype(P.ty, "a scalar") +
             ")p" + std::to_string(i) + ";");
    }
    for (int a = 2; a >= 0; --a) {
      line("for (long long blk" + std::to_string(a) + " = 0; blk" + std::to_string(a) + " < " +
           std::to_string(K.launch.grid[a]) + "; ++blk" + std::to_string(a) + ") {");
      ++depth;
    }
    for (size_t i = 0; i < K.allocs.size(); ++i) {
      const Alloc& A = K.allocs[i];
      const long long len = A.space == "Private" ? A.extent * K.launch.threads() : A.extent;
      line(std::string(ctype(A.elem, "an allocation")) + " sh" + std::to_string(i) + "[" + std::to_string(len) + "] = {0};");
    }
    phases(*K.body);
    for (int a = 0; a < 3; ++a) {
      --depth;
      line("}");
    }
  }

  void serial_body() {
    for (size_t i = 0; i < K.params.size(); ++i) {
      const Param& P = K.params[i];
      if (!P.buffer) {
        const std::string t = ctype(P.ty, "a scalar");
        line(t + " l" + std::to_string(P.local) + " = p" + std::to_string(i) + ";");
      }
    }
    block(*K.body);
  }

  std::string signature(const std::string& fname) const {
    std::string s = "int " + fname + "(";
    bool first = true;
    auto arg = [&](const std::string& a) {
      s += first ? "\n    " : ",\n    ";
      s += a;
      first = false;
    };
    for (size_t i = 0; i < K.params.size(); ++i) {
      const Param& P = K.params[i];
      const std::string b = "b" + std::to_string(i);
      if (P.buffer) {
        const std::string base = is_subbyte(P.elem) ? "unsigned char" : ctype(P.elem, "a buffer");
        const bool written = P.role == "Write" || P.role == "ReadWrite";
        arg((written ? "" : "const ") + base + "* " + b);
        arg("const long long* " + b + "_shape");
        arg("const long long* " + b + "_stride");
        arg("long long " + b + "_base");
      } else {
        arg(std::string(ctype(P.ty, "a scalar")) + " p" + std::to_string(i));
      }
    }
    if (first) s += "void";
    return s + ")";
  }
};

// ---- the prelude: helpers the spellings call ------------------------------------------------------
// The semantics are the C leg's (typed.rs:27-76, narrow.rs, cfamily.rs:223-304); the text is this
// file's own.  Float to integer: a NaN gives 0 and a value past either end of the kind the nearer
// end (the caller has rounded it already).  Integer Div, Shl, Shr by the total rule: a zero divisor
// gives the dividend, a signed divisor of -1 negates with wrap (MIN / -1 is MIN), a shift count's
// bits are taken modulo the width, and >> on a signed kind fills with the sign bit.
const char* kTypedHelpers = R"(static long long leg_f2i_sat(double y, long long lo, long long hi) {
    if (y != y) return 0;
    if (y <= (double)lo) return lo;
    if (y >= (double)hi) return hi;
    return (long long)y;
}
static long long leg_clamp(long long v, long long lo, long long hi) {
    if (v < lo) return lo;
    return v > hi ? hi : v;
}
#define LEG_SIGNED_OPS(S, T, U, W) \
static T leg_div_##S(T a, T b) { \
    if (b == 0) return a; \
    if (b == (T)-1) return (T)((U)0 - (U)a); \
    return a / b; \
} \
static T leg_shl_##S(T a, T c) { return (T)((U)a << ((U)c & (U)(W - 1))); } \
static T leg_shr_##S(T a, T c) { \
    const U k = (U)c & (U)(W - 1); \
    const U sign_fill = a < 0 ? ~(~(U)0 >> k) : (U)0; \
    return (T)(((U)a >> k) | sign_fill); \
}
#define LEG_UNSIGNED_OPS(S, U, W) \
static U leg_div_##S(U a, U b) { return b == 0 ? a : a / b; } \
static U leg_shl_##S(U a, U c) { return a << (c & (U)(W - 1)); } \
static U leg_shr_##S(U a, U c) { return a >> (c & (U)(W - 1)); }
LEG_SIGNED_OPS(i32, int, unsigned int, 32)
LEG_SIGNED_OPS(i64, long long, unsigned long long, 64)
LEG_UNSIGNED_OPS(u32, unsigned int, 32)
LEG_UNSIGNED_OPS(u64, unsigned long long, 64)
)";

// The 16-bit float codec for a binary format of `eb` exponent bits and `mb` fraction bits (F16: 5, 10;
// Bf16: 8, 7).  Decoding is exact.  Encoding rounds a double once, to nearest with ties to even: the
// magnitude is scaled by a power of two (exact) to units of its binade's quantum (the subnormal
// quantum below the normal range), rounded to an integer in the default rounding mode, and the
// integer's bits become the fraction; a count reaching the next binade carries into the exponent
// field, and past the largest finite value the result is infinity.  A NaN encodes as the quiet NaN
// with its sign.
const char* kCodec = R"(static unsigned leg_encode(double x, int eb, int mb) {
    const unsigned sign = signbit(x) ? 1u << (eb + mb) : 0u, inf = ((1u << eb) - 1u) << mb;
    const int bias = (1 << (eb - 1)) - 1, emin = 1 - bias;
    double a = fabs(x), units;
    unsigned long long n;
    unsigned body;
    int e;
    if (a != a) return sign | inf | (1u << (mb - 1));
    if (a == 0.0) return sign;
    if (isinf(a)) return sign | inf;
    (void)frexp(a, &e);
    e -= 1;
    if (e < emin) e = emin;
    if (e > bias) return sign | inf;
    units = nearbyint(ldexp(a, mb - e));
    n = (unsigned long long)units;
    if (e == emin && n < (1ull << mb)) body = (unsigned)n;
    else body = ((unsigned)(e + bias) << mb) + (unsigned)(n - (1ull << mb));
    return sign | (body >= inf ? inf : body);
}
static double leg_decode(unsigned h, int eb, int mb) {
    const int bias = (1 << (eb - 1)) - 1;
    const unsigned field = (h >> mb) & ((1u << eb) - 1u), frac = h & ((1u << mb) - 1u);
    double v;
    if (field == (1u << eb) - 1u) v = frac ? NAN : INFINITY;
    else if (field == 0) v = ldexp((double)frac, 1 - bias - mb);
    else v = ldexp((double)(frac | (1u << mb)), (int)field - bias - mb);
    return (h >> (eb + mb)) & 1u ? -v : v;
}
static unsigned short leg_to_bf16(double x) { return (unsigned short)leg_encode(x, 8, 7); }
static unsigned short leg_to_f16(double x) { return (unsigned short)leg_encode(x, 5, 10); }
static float leg_bf16_value(unsigned short h) {
    /* a Bf16 is the upper half of an F32: the bits move, NaN payloads included */
    const unsigned int w = (unsigned int)h << 16;
    float f;
    memcpy(&f, &w, sizeof f);
    return f;
}
static float leg_f16_value(unsigned short h) { return (float)leg_decode(h, 5, 10); }
)";

std::string ident(const std::string& x) {
  std::string s = x;
  for (char& c : s)
    if (!isalnum((unsigned char)c)) c = '_';
  return s;
}

std::string lower(const V& k, std::string& entry) {
  Kernel K = read_kernel(k);
  admit(K);
  Emitter em(K);
  if (K.launched)
    em.launched_body();
  else
    em.serial_body();
  entry = "unpopped_cpu_kernel_" + ident(K.name);
  const std::string body = em.signature(entry) + " {\n" + em.out + "    return 0;\n}\n";
  std::string src = "/* Generated by the cpu-c restatement (serial C99): do not edit. kernel: " + K.name + " */\n";
  src += "#include <math.h>\n#include <string.h>\n\n";
  src += kTypedHelpers;
  if (body.find("leg_to_") != std::string::npos || body.find("_value(") != std::string::npos) src += kCodec;
  return src + "\n" + body;
}

char* dup(const std::string& s) {
  char* p = (char*)malloc(s.size() + 1);
  memcpy(p, s.c_str(), s.size() + 1);
  return p;
}

}  // namespace

extern "C" {

// Lower a KernelFn (its serde JSON) to C99.  Returns 0 with the source and the entry-point name,
// 6 (LowerError::UnsupportedKernel, crates/unpopped/src/backend.rs:436) with the reason, or 50 for
// text that is not JSON.  Strings are freed with cpuc_free.
int cpuc_lower_kernel(const char* json, char** source, char** entry, char** detail) {
  *source = *entry = *detail = nullptr;
  Reader r{json, json + strlen(json), {}};
  V k;
  if (!r.val(k, 0)) {
    *detail = dup("cpu_c: not JSON: " + r.err);
    return 50;
  }
  try {
    std::string name;
    std::string src = lower(k, name);
    *source = dup(src);
    *entry = dup(name);
    return 0;
  } catch (const Refuse& e) {
    *detail = dup("cpu_c: " + e.why);
    return 6;
  }
}

void cpuc_free(char* p) { free(p); }
}
