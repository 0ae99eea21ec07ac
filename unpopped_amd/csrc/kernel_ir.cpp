// JSON value tree of a KernelFn: parser, writer, structural equality and serde-shaped builders.
#include "kernel_ir.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>

namespace unp {
namespace kir {

const J* J::get(const std::string& key) const {
  if (t != Obj) return nullptr;
  for (const auto& kv : o)
    if (kv.first == key) return &kv.second;
  return nullptr;
}

bool J::operator==(const J& x) const {
  if (t != x.t) return false;
  switch (t) {
    case Null:
      return true;
    case Bool:
      return b == x.b;
    case Num:
      if (is_int && x.is_int) return i == x.i;
      return d == x.d;
    case Str:
      return s == x.s;
    case Arr:
      if (a.size() != x.a.size()) return false;
      for (size_t k = 0; k < a.size(); ++k)
        if (!(a[k] == x.a[k])) return false;
      return true;
    case Obj: {
      if (o.size() != x.o.size()) return false;
      for (const auto& kv : o) {
        const J* other = x.get(kv.first);
        if (!other || !(kv.second == *other)) return false;
      }
      return true;
    }
  }
  return false;
}

namespace {

struct Parser {
  const std::string& s;
  size_t p = 0;
  std::string err;
  int depth = 0;

  void ws() {
    while (p < s.size() && (s[p] == ' ' || s[p] == '\n' || s[p] == '\r' || s[p] == '\t')) ++p;
  }
  bool fail(const std::string& m) {
    if (err.empty()) err = m + " at byte " + std::to_string(p);
    return false;
  }
  bool lit(const char* w) {
    size_t n = std::char_traits<char>::length(w);
    if (s.compare(p, n, w) != 0) return false;
    p += n;
    return true;
  }
  bool value(J& out) {
    if (++depth > 512) return fail("nesting too deep");
    ws();
    if (p >= s.size()) return fail("unexpected end");
    const char c = s[p];
    bool ok = false;
    if (c == '{') ok = object(out);
    else if (c == '[') ok = array(out);
    else if (c == '"') {
      out = J::str("");
      ok = string(out.s);
    } else if (lit("null")) {
      out = J::null();
      ok = true;
    } else if (lit("true")) {
      out = J::boolean(true);
      ok = true;
    } else if (lit("false")) {
      out = J::boolean(false);
      ok = true;
    } else ok = number(out);
    --depth;
    return ok;
  }
  bool string(std::string& out) {
    if (s[p] != '"') return fail("expected a string");
    ++p;
    while (p < s.size() && s[p] != '"') {
      char c = s[p++];
      if (c == '\\') {
        if (p >= s.size()) return fail("bad escape");
        const char e = s[p++];
        switch (e) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            if (p + 4 > s.size()) return fail("bad \\u escape");
            const unsigned cp = (unsigned)std::strtoul(s.substr(p, 4).c_str(), nullptr, 16);
            p += 4;
            if (cp < 0x80) out += (char)cp;
            else if (cp < 0x800) {
              out += (char)(0xC0 | (cp >> 6));
              out += (char)(0x80 | (cp & 0x3F));
            } else {
              out += (char)(0xE0 | (cp >> 12));
              out += (char)(0x80 | ((cp >> 6) & 0x3F));
              out += (char)(0x80 | (cp & 0x3F));
            }
            break;
          }
          default:
            return fail("bad escape");
        }
      } else {
        out += c;
      }
    }
    if (p >= s.size()) return fail("unterminated string");
    ++p;
    return true;
  }
  bool number(J& out) {
    const size_t start = p;
    bool integral = true;
    if (p < s.size() && (s[p] == '-' || s[p] == '+')) ++p;
    while (p < s.size()) {
      const char c = s[p];
      if (c >= '0' && c <= '9') {
        ++p;
      } else if (c == '.' || c == 'e' || c == 'E' || c == '-' || c == '+') {
        integral = false;
        ++p;
      } else {
        break;
      }
    }
    if (p == start) return fail("unexpected character");
    const std::string tok = s.substr(start, p - start);
    char* end = nullptr;
    if (integral) {
      errno = 0;
      const long long v = std::strtoll(tok.c_str(), &end, 10);
      if (end && *end == '\0' && errno == 0) {
        out = J::integer(v);
        return true;
      }
    }
    const double v = std::strtod(tok.c_str(), &end);
    if (!end || *end != '\0') return fail("bad number");
    out = J::number(v);
    return true;
  }
  bool array(J& out) {
    out = J::arr();
    ++p;
    ws();
    if (p < s.size() && s[p] == ']') {
      ++p;
      return true;
    }
    for (;;) {
      J v;
      if (!value(v)) return false;
      out.a.push_back(std::move(v));
      ws();
      if (p < s.size() && s[p] == ',') {
        ++p;
        continue;
      }
      if (p < s.size() && s[p] == ']') {
        ++p;
        return true;
      }
      return fail("expected , or ]");
    }
  }
  bool object(J& out) {
    out = J::obj();
    ++p;
    ws();
    if (p < s.size() && s[p] == '}') {
      ++p;
      return true;
    }
    for (;;) {
      ws();
      std::string k;
      if (p >= s.size() || !string(k)) return fail("expected a key");
      ws();
      if (p >= s.size() || s[p] != ':') return fail("expected :");
      ++p;
      J v;
      if (!value(v)) return false;
      out.o.emplace_back(std::move(k), std::move(v));
      ws();
      if (p < s.size() && s[p] == ',') {
        ++p;
        continue;
      }
      if (p < s.size() && s[p] == '}') {
        ++p;
        return true;
      }
      return fail("expected , or }");
    }
  }
};

void write_to(const J& j, std::string& o) {
  switch (j.t) {
    case J::Null:
      o += "null";
      break;
    case J::Bool:
      o += j.b ? "true" : "false";
      break;
    case J::Num: {
      char buf[64];
      if (j.is_int) {
        std::snprintf(buf, sizeof buf, "%lld", (long long)j.i);
      } else if (std::isfinite(j.d) && j.d == std::floor(j.d) && std::fabs(j.d) < 1e15) {
        std::snprintf(buf, sizeof buf, "%.1f", j.d);
      } else {
        std::snprintf(buf, sizeof buf, "%.17g", j.d);
      }
      o += buf;
      break;
    }
    case J::Str:
      o += '"';
      for (char c : j.s) {
        if (c == '"' || c == '\\') {
          o += '\\';
          o += c;
        } else if (c == '\n') {
          o += "\\n";
        } else {
          o += c;
        }
      }
      o += '"';
      break;
    case J::Arr:
      o += '[';
      for (size_t k = 0; k < j.a.size(); ++k) {
        if (k) o += ',';
        write_to(j.a[k], o);
      }
      o += ']';
      break;
    case J::Obj:
      o += '{';
      for (size_t k = 0; k < j.o.size(); ++k) {
        if (k) o += ',';
        o += '"';
        o += j.o[k].first;
        o += "\":";
        write_to(j.o[k].second, o);
      }
      o += '}';
      break;
  }
}

}  // namespace

bool parse(const std::string& text, J& out, std::string& err) {
  Parser ps{text};
  if (!ps.value(out)) {
    err = ps.err;
    return false;
  }
  ps.ws();
  if (ps.p != text.size()) {
    err = "trailing characters at byte " + std::to_string(ps.p);
    return false;
  }
  return true;
}

std::string write(const J& j) {
  std::string o;
  write_to(j, o);
  return o;
}

// ---- builders ---------------------------------------------------------------------------

J e_const(double v) {
  if (std::isnan(v)) return var("Const", J::str("NaN"));
  if (std::isinf(v)) return var("Const", J::str(v > 0 ? "inf" : "-inf"));
  return var("Const", J::number(v));
}
J e_int(int64_t v, const char* ek) { return tup("ConstInt", {J::integer(v), J::str(ek)}); }
J e_local(uint32_t l) { return var("Local", J::integer(l)); }
J e_exec(const char* id, int axis) {
  return var("Exec", axis < 0 ? unit(id) : var(id, J::integer(axis)));
}
J e_add(J a, J b) { return tup("Add", {std::move(a), std::move(b)}); }
J e_sub(J a, J b) { return tup("Sub", {std::move(a), std::move(b)}); }
J e_mul(J a, J b) { return tup("Mul", {std::move(a), std::move(b)}); }
J e_div(J a, J b) { return tup("Div", {std::move(a), std::move(b)}); }
J e_bin(const char* op, J a, J b) { return tup("Binary", {J::str(op), std::move(a), std::move(b)}); }
J e_cast(J a, const char* to, const char* round, const char* sat) {
  return tup("Cast", {std::move(a), J::obj({{"to", J::str(to)}, {"round", J::str(round)}, {"sat", J::str(sat)}})});
}
J e_bitcast(J a, const char* to) { return tup("Bitcast", {std::move(a), J::str(to)}); }

J p_logical(uint32_t buffer, std::vector<J> coords) {
  return var("Logical", J::obj({{"buffer", J::integer(buffer)}, {"coords", J::arr(std::move(coords))}}));
}
J p_alloc(uint32_t alloc, J index) {
  return var("Alloc", J::obj({{"alloc", J::integer(alloc)}, {"index", std::move(index)}}));
}
J s_let(uint32_t local, J init) { return var("Let", J::obj({{"local", J::integer(local)}, {"init", std::move(init)}})); }
J s_load(uint32_t local, J place) {
  return var("Load", J::obj({{"local", J::integer(local)}, {"place", std::move(place)}}));
}
J s_assign(uint32_t local, J value) {
  return var("Assign", J::obj({{"local", J::integer(local)}, {"value", std::move(value)}}));
}
J s_store(J place, J value) { return var("Store", J::obj({{"place", std::move(place)}, {"value", std::move(value)}})); }
J s_if(J cond, std::vector<J> then, std::vector<J> els) {
  return var("If", J::obj({{"cond", std::move(cond)}, {"then", J::arr(std::move(then))}, {"els", J::arr(std::move(els))}}));
}
J s_for(uint32_t local, J start, J end, J step, std::vector<J> body) {
  return var("For", J::obj({{"local", J::integer(local)},
                            {"start", std::move(start)},
                            {"end", std::move(end)},
                            {"step", std::move(step)},
                            {"unroll", unit("None")},
                            {"body", J::arr(std::move(body))}}));
}
J s_while(J cond, std::vector<J> body) {
  return var("While", J::obj({{"cond", std::move(cond)}, {"body", J::arr(std::move(body))}}));
}
J s_barrier() { return var("Barrier", J::obj({{"scope", unit("Block")}, {"kind", unit("Full")}})); }

J param_buffer(const std::string& name, const char* elem, const char* role, int rank) {
  return J::obj({{"name", J::str(name)},
                 {"kind", var("Buffer", J::obj({{"elem", J::str(elem)},
                                                {"role", J::str(role)},
                                                {"rank", rank < 0 ? J::null() : J::integer(rank)}}))}});
}
J param_scalar(const std::string& name, const char* ty, uint32_t local) {
  return J::obj({{"name", J::str(name)}, {"kind", var("Scalar", J::obj({{"ty", J::str(ty)}, {"local", J::integer(local)}}))}});
}
J local_decl(const char* elem) { return J::obj({{"elem", J::str(elem)}, {"lanes", J::integer(1)}}); }
J launch_shape(uint32_t block, uint32_t grid) {
  return J::obj({{"block", J::arr({J::integer(block), J::integer(1), J::integer(1)})},
                 {"grid", J::arr({J::integer(grid), J::integer(1), J::integer(1)})},
                 {"subgroup", J::null()},
                 {"cluster", J::null()},
                 {"devices", J::integer(1)},
                 {"grid_dims", J::null()}});
}
J alloc_shared(const char* name, const char* elem, uint32_t extent) {
  return J::obj({{"name", J::str(name)},
                 {"space", unit("Shared")},
                 {"elem", J::str(elem)},
                 {"extent", var("Static", J::integer(extent))}});
}
J kernel_fn(const std::string& name, const char* compute, std::vector<J> params, std::vector<J> locals,
            std::vector<J> body, J launch, std::vector<J> allocs) {
  return J::obj({{"name", J::str(name)},
                 {"compute", J::str(compute)},
                 {"params", J::arr(std::move(params))},
                 {"locals", J::arr(std::move(locals))},
                 {"body", J::arr(std::move(body))},
                 {"launch", std::move(launch)},
                 {"allocs", J::arr(std::move(allocs))},
                 {"result", J::null()},
                 {"results", J::arr()}});
}

}  // namespace kir
}  // namespace unp
