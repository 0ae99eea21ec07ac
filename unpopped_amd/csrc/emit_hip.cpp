// The HIP emitter: one lowered form -> kernel source (the device template library plus the
// `extern "C"` entry points that instantiate it) and the launch interface as JSON.
//
// The emitted text is what GeneratedKernel::source carries (crates/unpopped/src/backend.rs
// :105-125); the interface JSON carries the KernelInterface fields the launch needs
// (crates/unpopped/src/kernel_interface.rs:200-237): launch geometry, parameters, entry
// symbols, launch bounds, compiler arguments and fidelity notes.
#include <sstream>

#include "unp_internal.hpp"

namespace unp {

extern const char* const kDeviceLibrary;  // unp_device.hip, embedded at build time

namespace {

struct KindInfo {
  int32_t kind;
  const char* name;
  size_t bytes;
};

const KindInfo kKinds[] = {
    {UNP_F16, "F16", 2},       {UNP_BF16, "Bf16", 2},
    {UNP_F32, "F32", 4},       {UNP_F32_STRICT, "F32Strict", 4},
    {UNP_F64, "F64", 8},       {UNP_I8, "I8", 1},
    {UNP_I16, "I16", 2},       {UNP_U8, "U8", 1},
    {UNP_U16, "U16", 2},       {UNP_I32, "I32", 4},
    {UNP_I64, "I64", 8},       {UNP_BOOL, "Bool", 1},
    {UNP_FP8_E4M3FN, "Fp8E4M3FN", 1},   {UNP_FP8_E4M3FNUZ, "Fp8E4M3FNUZ", 1},
    {UNP_FP8_E5M2, "Fp8E5M2", 1},       {UNP_F8_E8M0, "F8E8M0", 1},
    {UNP_F8_E6M2, "F8E6M2", 1},         {UNP_FP8_E5M2FNUZ, "Fp8E5M2FNUZ", 1},
    {UNP_I4, "I4", 0},         {UNP_U4, "U4", 0},
    {UNP_B1, "B1", 0},         {UNP_COMPLEX64, "Complex64", 8},
    {UNP_COMPLEX128, "Complex128", 16}, {UNP_U32, "U32", 4},
    {UNP_U64, "U64", 8},       {UNP_F4_E2M1, "F4E2M1", 0},
    {UNP_F6_E2M3, "F6E2M3", 0}, {UNP_F6_E3M2, "F6E3M2", 0},
};

const char* op_name(int32_t op) {
  switch (op) {
    case UNP_OP_SUM: return "sum";
    case UNP_OP_PROD: return "prod";
    case UNP_OP_MAX: return "max";
    case UNP_OP_MIN: return "min";
    case UNP_OP_MEAN: return "mean";
    case UNP_OP_AND: return "and";
    case UNP_OP_OR: return "or";
    case UNP_OP_XOR: return "xor";
    case UNP_OP_MAXNUM: return "maxnum";
    case UNP_OP_MINNUM: return "minnum";
    default: return nullptr;
  }
}

const char* oob_name(int32_t p) {
  switch (p) {
    case UNP_OOB_SKIP: return "Skip";
    case UNP_OOB_ZEROFILL: return "ZeroFill";
    case UNP_OOB_CLAMP: return "Clamp";
    default: return nullptr;
  }
}

// The C++ element type the device library instantiates for a compute kind.
const char* ctype(int32_t kind) {
  switch (kind) {
    case UNP_F32: return "float";
    case UNP_F64: return "double";
    case UNP_I32: return "int";
    case UNP_I64: return "long long";
    case UNP_U32: return "unsigned int";
    default: return nullptr;
  }
}

const char* lower_name(int32_t kind) {
  switch (kind) {
    case UNP_F32: return "f32";
    case UNP_F64: return "f64";
    case UNP_I32: return "i32";
    case UNP_I64: return "i64";
    case UNP_U32: return "u32";
    case UNP_U64: return "u64";
    case UNP_I16: return "i16";
    case UNP_U16: return "u16";
    case UNP_BF16: return "bf16";
    case UNP_F16: return "f16";
    case UNP_U4: return "u4";
    case UNP_I4: return "i4";
    case UNP_I8: return "i8";
    case UNP_U8: return "u8";
    default: return "x";
  }
}

std::string json_str(const std::string& s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += c;
    } else if (c == '\n') {
      o += "\\n";
    } else {
      o += c;
    }
  }
  return o + "\"";
}

// The folds the reduction forms accept at F32/F64/I32/I64 (kernel_lift.rs:763-803): those of
// lift_reduction_opdef_launched (crates/unpopped/src/kernel_lift/block_reduce.rs:97-133), float
// Sum/Mean/Max/Min and integer Sum/Prod/Max/Min, and the sequential lift's MaxNum/MinNum and integer
// And/Or/Xor, whose results do not depend on the fold's order (NaN payload and the sign of a zero
// tie aside, as for Max/Min).
bool reduction_ok(int32_t dtype, int32_t op, std::string& why) {
  if (!ctype(dtype) || dtype == UNP_U32) {
    why = "a reduction outside F32, F64, I32 and I64";
    return false;
  }
  if (!op_name(op)) {
    why = "a reduce op this backend has no fold for";
    return false;
  }
  const bool is_int = kind_is_int(dtype);
  if (is_int && op == UNP_OP_MEAN) {
    why = "an integer Mean";
    return false;
  }
  if (!is_int && (op == UNP_OP_AND || op == UNP_OP_OR || op == UNP_OP_XOR)) {
    why = "a bit reduction at a float dtype";
    return false;
  }
  return true;
}

int vec_of(int32_t dtype) { return 16 / (int)kind_bytes(dtype); }

std::string header(const std::string& name, const unp_form& f) {
  std::ostringstream s;
  s << "// unpopped-hip kernel `" << name << "` for rocm:gfx950 (form " << f.kind << ").\n";
  s << kDeviceLibrary << "\n";
  return s.str();
}

const char* kLaunchBounds = "__launch_bounds__(256)";

}  // namespace

const char* kind_name(int32_t kind) {
  for (const auto& k : kKinds)
    if (k.kind == kind) return k.name;
  return nullptr;
}

int32_t kind_from_name(const std::string& s) {
  for (const auto& k : kKinds)
    if (s == k.name) return k.kind;
  return -1;
}

size_t kind_bytes(int32_t kind) {
  for (const auto& k : kKinds)
    if (k.kind == kind) return k.bytes;
  return 0;
}

bool kind_is_float(int32_t kind) {
  return kind == UNP_F32 || kind == UNP_F64 || kind == UNP_F16 || kind == UNP_BF16 ||
         kind == UNP_F32_STRICT;
}
bool kind_is_int(int32_t kind) {
  return kind == UNP_I32 || kind == UNP_I64 || kind == UNP_U32 || kind == UNP_I8 ||
         kind == UNP_I16 || kind == UNP_U8 || kind == UNP_U16 || kind == UNP_U64;
}

uint64_t fnv1a64(const std::string& s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 0x00000100000001b3ull;
  }
  return h;
}

void set_error(unp_error* err, int32_t code, const std::string& detail) {
  if (!err) return;
  err->code = code;
  std::snprintf(err->detail, sizeof(err->detail), "%s", detail.c_str());
}

uint32_t reduction_mask(const unp_form& f) {
  if (f.axes_mask) return f.axes_mask;
  uint32_t m = 0;
  for (int32_t d = f.reduced_from; d < f.rank; ++d) m |= 1u << d;
  return m;
}

char reduction_schedule(uint32_t mask, int32_t rank) {
  std::string runs;  // one letter per run of adjacent axes of a kind
  for (int32_t d = 0; d < rank; ++d) {
    const char c = (mask >> d) & 1u ? 'R' : 'K';
    if (runs.empty() || runs.back() != c) runs.push_back(c);
  }
  if (runs == "R") return 'a';
  if (runs == "KR") return 'r';
  if (runs == "RK" || runs == "KRK") return 'm';
  return 'g';
}

// When the executor picks an entry that reads through storage-image strides.
static const char* const kStridedWhen =
    "a storage image that is not dense row-major (unp_hip_exec_launch_views): the view's strides";

static int32_t lower_reduction(const unp_form& f, Lowered& L, std::string& why) {
  const bool two = f.kind == UNP_FORM_ROW_REDUCE2;
  if (f.rank < 1 || f.rank > 8) {
    why = "rank is zero or more than 8";
    return UNP_LIFT_DECLINE;
  }
  const uint32_t mask = reduction_mask(f);
  if (mask == 0 || (mask >> f.rank) != 0) {
    why = "a reduced axis outside the rank";
    return UNP_LIFT_DECLINE;
  }
  // A float Prod has no order-free form and no declared bound: it runs in the serial lift's own
  // order (the launched lift refuses it, block_reduce.rs:97-133); so does every reduction asked
  // for on the serial schedule.
  if (two && f.schedule == UNP_SCHEDULE_SERIAL) {
    why = "the fused row fold has no serial schedule (its default is the device schedule)";
    return UNP_UNSUPPORTED_SCHEDULE;
  }
  const bool serial = (kind_is_float(f.dtype) && f.op0 == UNP_OP_PROD) || f.schedule == UNP_SCHEDULE_SERIAL;
  const char sched = serial ? 'q' : reduction_schedule(mask, f.rank);
  if (two && sched != 'r') {
    why = "the fused row fold reduces the trailing axis";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (two && kind_is_float(f.dtype) && f.op1 == UNP_OP_PROD) {
    why = "a float Prod in the fused row fold (not order-independent, and no declared bound)";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (!reduction_ok(f.dtype, f.op0, why) || (two && !reduction_ok(f.dtype, f.op1, why)))
    return UNP_UNSUPPORTED_KERNEL;
  const char* T = ctype(f.dtype);
  const int V = vec_of(f.dtype);
  L.axes_mask = mask;
  L.red_schedule = sched;
  L.reduce_all = sched == 'a';
  L.form.reduced_from = f.rank;
  for (int32_t d = f.rank - 1; d >= 0 && ((mask >> d) & 1u); --d) L.form.reduced_from = d;
  std::ostringstream name;
  name << (sched == 'a'   ? "unp_reduce_all_"
           : sched == 'm' ? "unp_reduce_mid_"
           : sched == 'g' ? "unp_reduce_axes_"
           : sched == 'q' ? "unp_reduce_serial_"
                          : "unp_rowreduce_")
       << op_name(f.op0);
  if (two) name << "_" << op_name(f.op1);
  name << "_" << lower_name(f.dtype);
  L.name = name.str();
  std::ostringstream src;
  src << header(L.name, f);
  if (sched == 'm') {
    // Eight waves per block, one block per CU, 8 rows in flight per lane; blocks split the
    // reduced extent so that a launch has about cu_count blocks (measured best for an
    // 8192 x 4096 f32 column sum: more chunks cost more in the partials' final fold than they
    // add in parallelism).
    L.threads = 512;
    L.blocks_per_cu = 1;
    for (int fast = 1; fast >= 0; --fast) {
      Entry e;
      e.fast = fast;
      e.vec = fast ? V : 1;
      e.symbol = L.name + (fast ? "_mv" : "_ms");
      src << "extern \"C\" __global__ void __launch_bounds__(512) " << e.symbol << "(const " << T << "* in, " << T
          << "* out, long long A, long long R, long long B, long long S, "
          << "unsigned long long* partials, unsigned* counters, unsigned epoch, unp::waits wt) {\n  unp::reduce_mid<" << T
          << ", " << f.op0 << ", " << e.vec << ", 512, 8>(in, out, A, R, B, S, partials, counters, epoch, wt);\n}\n";
      L.entries.push_back(e);
    }
  } else if (sched == 'q') {
    L.threads = 256;
    L.blocks_per_cu = 8;
    Entry e;
    e.fast = false;
    e.vec = 1;
    e.symbol = L.name + "_q";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(const " << T << "* in, " << T
        << "* out, unp::red_view d) {\n  unp::reduce_serial<" << T << ", " << f.op0 << ", 256>(in, out, d);\n}\n";
    L.entries.push_back(e);
  } else if (sched == 'g') {
    L.threads = 256;
    L.blocks_per_cu = 8;
    Entry e;
    e.fast = false;
    e.vec = 1;
    e.symbol = L.name + "_g";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(const " << T << "* in, " << T
        << "* out, unp::axes_desc d) {\n  unp::reduce_generic<" << T << ", " << f.op0 << ", 256>(in, out, d);\n}\n";
    L.entries.push_back(e);
  } else if (L.reduce_all) {
    // One block per CU (8 waves): the read rate peaks with few streams per CU.
    L.threads = 512;
    L.blocks_per_cu = 1;
    for (int fast = 1; fast >= 0; --fast) {
      Entry e;
      e.fast = fast;
      e.vec = fast ? V : 1;
      e.symbol = L.name + (fast ? "_v" : "_s");
      src << "extern \"C\" __global__ void __launch_bounds__(512) " << e.symbol << "(const " << T << "* in, " << T
          << "* out, long long n, unsigned long long* partials, unsigned* counter, unsigned epoch, unp::waits wt) {\n"
          << "  unp::reduce_all<" << T << ", " << f.op0 << ", " << e.vec << ", 512, " << (fast ? 16 : 8)
          << ">(in, out, n, partials, counter, epoch, wt);\n}\n";
      L.entries.push_back(e);
    }
  } else {
    // Rows up to kWideRow (32768) elements: one wave per row (no barrier); longer rows: one
    // block per row with the LDS combine.  Both read the row once and stream it past the caches.
    // Two blocks of four waves per CU (measured best for an 8192 x 4096 f32 row read).
    L.threads = 256;
    L.blocks_per_cu = 2;
    for (int wide = 0; wide <= 1; ++wide) {
      for (int fast = 1; fast >= 0; --fast) {
        Entry e;
        e.fast = fast;
        e.wide = wide;
        e.vec = fast ? V : 1;
        e.symbol = L.name + (wide ? "_b" : "_w") + (fast ? "v" : "s");
        const int unroll = wide ? (fast ? 4 : 8) : 16;
        src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(const " << T << "* in, " << T
            << "* out0, " << T << "* out1, long long rows, long long cols) {\n  unp::"
            << (wide ? "rowreduce<" : "rowreduce_wave<") << T << ", " << f.op0 << ", " << (two ? f.op1 : f.op0) << ", "
            << (two ? 2 : 1) << ", " << e.vec << ", 256, " << unroll << ">(in, out0, out1, rows, cols);\n}\n";
        L.entries.push_back(e);
      }
    }
  }
  // Storage images that are not dense row-major (transposed, strided, reversed): one wave per
  // output reading through the view's strides (the serial product: one lane per output, its own
  // order); the fused row fold runs one launch per fold.
  for (int o = 0; o < (two ? 2 : 1); ++o) {
    Entry e;
    e.strided = true;
    e.vec = 1;
    e.threads = 256;
    e.blocks_per_cu = 8;
    e.symbol = L.name + (o ? "_x1" : "_x");
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(const " << T << "* in, " << T
        << "* out, unp::red_view v) {\n  unp::";
    if (sched == 'q') src << "reduce_serial<" << T << ", " << f.op0 << ", 256>(in, out, v);\n}\n";
    else src << "reduce_strided<" << T << ", " << (o ? f.op1 : f.op0) << ", 256>(in, out, v);\n}\n";
    L.entries.push_back(e);
  }
  L.source = src.str();
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":"
    << (two ? "\"row_reduce2\"" : "\"reduction\"") << ",\"dtype\":\"" << kind_name(f.dtype)
    << "\",\"ops\":[\"" << op_name(f.op0) << "\"" << (two ? std::string(",\"") + op_name(f.op1) + "\"" : "")
    << "],\"rank\":" << f.rank << ",\"reduced_axes\":[";
  for (int32_t d = 0, n = 0; d < f.rank; ++d)
    if ((mask >> d) & 1u) j << (n++ ? "," : "") << d;
  j << "],\"schedule\":\""
    << (sched == 'a' ? "all" : sched == 'r' ? "rows" : sched == 'm' ? "mid" : sched == 'q' ? "serial" : "generic")
    << "\""
    << ",\"params\":[{\"name\":\"in0\",\"kind\":\"buffer\",\"role\":\"Read\"},"
    << (two ? "{\"name\":\"out0\",\"kind\":\"buffer\",\"role\":\"Write\"},{\"name\":\"out1\",\"kind\":\"buffer\",\"role\":\"Write\"}"
            : "{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\"}");
  for (int d = 0; d < f.rank; ++d) j << ",{\"name\":\"n" << d << "\",\"kind\":\"scalar\",\"dtype\":\"I32\"}";
  j << "],\"launch\":{\"block\":[" << L.threads << ",1,1],\"grid\":\"cu_count*" << L.blocks_per_cu
    << "\",\"grid_policy\":\"device-class constant; "
    << (sched == 'a'   ? "blocks stride over 16-byte vectors, last-ticket block folds the partials"
        : sched == 'm' ? "the input as A x R x B: a wave per 64 x vec columns, blocks split R into chunks, the "
                         "last-ticket block of a column strip folds the chunk partials in chunk order"
        : sched == 'g' ? "one wave per output element, lanes stride over the reduced positions"
        : sched == 'q' ? "one lane per output element, the reduced positions folded in the serial lift's "
                         "order (the serial accumulator, row-major over the reduced axes)"
                       : "waves stride over rows (one wave per row); rows longer than 32768 elements: one block per row")
    << "\"},\"entries\":[";
  for (size_t i = 0; i < L.entries.size(); ++i)
    j << (i ? "," : "") << "{\"symbol\":\"" << L.entries[i].symbol << "\",\"vec\":" << L.entries[i].vec
      << ",\"when\":\"" << (L.entries[i].wide ? "reduced extent > 32768; " : "")
      << (L.entries[i].strided ? kStridedWhen
          : (sched == 'g' || sched == 'q') ? "always"
          : sched == 'm' ? (L.entries[i].fast ? "B % vec == 0 and in0 16-byte aligned" : "otherwise")
                         : (L.entries[i].fast ? "reduced extent % vec == 0 and in0 16-byte aligned" : "otherwise"))
      << "\"}";
  j << "],\"workspace\":"
    << (L.reduce_all   ? "{\"partials\":\"grid * 8 bytes per 4-byte accumulator word (tagged with the launch epoch)\",\"counter\":4,\"stall\":4,\"host_state\":[\"epoch\"]}"
        : sched == 'm' ? "{\"partials\":\"strips * chunks * 64 * vec * 8 bytes per 4-byte accumulator word (tagged with the launch epoch)\",\"counters\":\"strips * 4\",\"stall\":4,\"host_state\":[\"epoch\"]}"
                       : "null")
    << ",\"compiler_args\":[\"--offload-arch=gfx950\",\"-O3\",\"-Xclang\",\"-target-feature\",\"-Xclang\",\"-packed-fp32-ops\"]"
    << ",\"fidelity_notes\":["
    << json_str(sched == 'q' ? "the serial lift's own order and accumulator: bit-exact against the serial kernel for every op"
                : kind_is_float(f.dtype) && (f.op0 == UNP_OP_SUM || f.op0 == UNP_OP_MEAN || (two && (f.op1 == UNP_OP_SUM || f.op1 == UNP_OP_MEAN)))
                    ? "float Sum/Mean: f64 accumulation in an order fixed by (grid, block=256, vector width); "
                      "within the declared bound gamma_(n-1)*sum|x| + 1/2 ulp, not the KernelFn's (block, grid) order"
                    : "order-independent fold: bit-exact against the serial kernel except NaN payload and the sign of a zero in Max/Min")
    << "," << json_str("the launch geometry is the device's (cu_count x blocks), not the KernelFn's LaunchShape")
    << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

// A scan's entry over storage images: one lane per column, the scanned axis walked in the serial
// lift's order through the views' strides.
static std::string scan_strided_entry(const unp_form& f, Lowered& L) {
  Entry e;
  e.strided = true;
  e.vec = 1;
  e.threads = 256;
  e.blocks_per_cu = 8;
  e.symbol = L.name + "_x";
  const char* T = ctype(f.dtype);
  std::ostringstream src;
  src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(const " << T << "* in, " << T
      << "* out, unp::scan_view v) {\n  unp::scan_strided<" << T << ", " << f.op0 << ", "
      << (f.exclusive ? "true" : "false") << ", " << (f.reverse ? "true" : "false") << ">(in, out, v);\n}\n";
  L.entries.push_back(e);
  return src.str();
}

static int32_t lower_scan(const unp_form& f, Lowered& L, std::string& why) {
  if (f.rank < 1 || f.rank > 8) {
    why = "rank is zero or more than 8";
    return UNP_LIFT_DECLINE;
  }
  if (!ctype(f.dtype) || f.dtype == UNP_U32) {
    why = "a scan outside F32, F64, I32 and I64";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (f.op0 != UNP_OP_SUM && f.op0 != UNP_OP_MAX && f.op0 != UNP_OP_MIN && f.op0 != UNP_OP_PROD &&
      f.op0 != UNP_OP_MEAN) {
    why = "a scan folds Sum, Prod, Max, Min or Mean";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (f.op0 == UNP_OP_MEAN && !kind_is_float(f.dtype)) {
    why = "an integer Mean";
    return UNP_UNSUPPORTED_KERNEL;
  }
  // The scanned axis: axes_mask's one bit, or the innermost axis.
  int32_t axis = f.rank - 1;
  if (f.axes_mask) {
    if ((f.axes_mask & (f.axes_mask - 1)) != 0 || (f.axes_mask >> f.rank) != 0) {
      why = "a scan scans exactly one axis inside the rank";
      return UNP_LIFT_DECLINE;
    }
    axis = __builtin_ctz(f.axes_mask);
  }
  // A non-innermost axis, or a float Prod (every product rounds, no declared bound), runs in the
  // serial lift's own order; so does every scan asked for on the serial schedule.
  const bool serial = axis != f.rank - 1 || (f.op0 == UNP_OP_PROD && kind_is_float(f.dtype)) ||
                      f.schedule == UNP_SCHEDULE_SERIAL;
  L.serial_scan = serial;
  L.scan_axis = axis;
  // The fixed schedule: a float fold's look-back combines tile aggregates in an association the
  // tiling alone fixes (lookback_grouped), so every launch gives the same bits.  An integer fold
  // gives the same bits in any order: its fixed schedule is the device schedule.
  const bool fixed = !serial && f.schedule == UNP_SCHEDULE_FIXED && kind_is_float(f.dtype);
  const char* T = ctype(f.dtype);
  std::ostringstream name;
  name << "unp_scan_" << (serial ? "seq_" : fixed ? "fix_" : "") << (f.exclusive ? "excl_" : "incl_")
       << (f.reverse ? "rev_" : "") << op_name(f.op0) << "_" << lower_name(f.dtype);
  L.name = name.str();
  if (serial) {
    Entry e;
    e.fast = false;
    e.vec = 1;
    e.threads = 256;
    e.blocks_per_cu = 8;
    e.symbol = L.name + "_q";
    std::ostringstream src;
    src << header(L.name, f);
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(const " << T << "* in, " << T
        << "* out, long long A, long long S, long long B) {\n  unp::scan_seq<" << T << ", " << f.op0 << ", "
        << (f.exclusive ? "true" : "false") << ", " << (f.reverse ? "true" : "false") << ", 8>(in, out, A, S, B);\n}\n";
    L.entries.push_back(e);
    src << scan_strided_entry(f, L);
    L.threads = 256;
    L.blocks_per_cu = 8;
    L.source = src.str();
    std::ostringstream j;
    j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"scan\",\"dtype\":\"" << kind_name(f.dtype)
      << "\",\"op\":\"" << op_name(f.op0) << "\",\"exclusive\":" << (f.exclusive ? "true" : "false")
      << ",\"reverse\":" << (f.reverse ? "true" : "false") << ",\"rank\":" << f.rank << ",\"axis\":" << axis
      << ",\"schedule\":\"serial\",\"params\":[{\"name\":\"in0\",\"kind\":\"buffer\",\"role\":\"Read\"},"
      << "{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\"}";
    for (int d = 0; d < f.rank; ++d) j << ",{\"name\":\"n" << d << "\",\"kind\":\"scalar\",\"dtype\":\"I32\"}";
    j << "],\"launch\":{\"block\":[256,1,1],\"grid\":\"cu_count*8\",\"grid_policy\":\"device-class constant; one "
      << "lane per column of the input seen as A x S x B around the scanned axis, lanes stride over columns\"},"
      << "\"entries\":[{\"symbol\":\"" << e.symbol << "\",\"when\":\"always\"},{\"symbol\":\""
      << L.entries.back().symbol << "\",\"when\":\"" << kStridedWhen << "\"}],\"workspace\":null"
      << ",\"compiler_args\":[\"--offload-arch=gfx950\",\"-O3\",\"-Xclang\",\"-target-feature\",\"-Xclang\",\"-packed-fp32-ops\"]"
      << ",\"fidelity_notes\":[" << json_str("the serial lift's own order: each column's prefix folds ascending (descending "
                                             "for a reverse scan) in the serial accumulator and rounds once per output; "
                                             "bit-exact against the serial scan")
      << "]}";
    L.interface_json = j.str();
    return UNP_OK;
  }
  // Two schedules, one ticket per block tile per round:
  //  _v  rows of a multiple of 16 bytes, 16-byte aligned: the LDS-staged scan, one producer
  //      wave streaming the next tile into LDS by DMA plus NC consumer waves, one block per
  //      CU (two LDS buffers of one 72 KiB tile each);
  //  _s  anything else: the register scan, one element per lane-vector.
  // Measured on MI355X at 2^28 i32 / 2^26 f32: a 4-byte carry runs best with 6 consumer waves
  // of K = 12 vectors, an 8-byte carry (f32 Sum in f64, F64, I64) on the device schedule with 4
  // waves of K = 18, and on the fixed schedule with 6 waves of K = 12 (its grouped look-back
  // starts sooner after the quicker in-tile scan: 121 against 131 us at 2^26 f32).
  const bool wide_carry = (f.dtype == UNP_F32 && f.op0 == UNP_OP_SUM) || kind_bytes(f.dtype) == 8;
  const bool wide_dev = wide_carry && !fixed;
  const int vec16 = vec_of(f.dtype);
  std::ostringstream src;
  src << header(L.name, f);
  {
    Entry e;
    e.fast = true;
    e.vec = vec16;
    e.k = wide_dev ? 18 : 12;
    e.wpb = wide_dev ? 4 : 6;  // consumer waves
    e.threads = 64 * (e.wpb + 1);
    e.blocks_per_cu = 1;
    e.symbol = L.name + "_v";
    src << "extern \"C\" __global__ void __launch_bounds__(" << e.threads << ") " << e.symbol << "(const " << T
        << "* in, " << T << "* out, long long rows, long long cols, unsigned long long* status, "
        << "unsigned* counter, unsigned ticket_base, unsigned epoch, unp::waits wt) {\n  unp::scan_staged<" << T << ", " << f.op0
        << ", " << (f.exclusive ? "true" : "false") << ", " << (f.reverse ? "true" : "false") << ", " << e.vec << ", "
        << e.k << ", " << e.wpb << ", " << kScanStatusWords << (fixed ? ", true" : "")
        << ">(in, out, rows, cols, status, counter, ticket_base, epoch, wt);\n}\n";
    L.entries.push_back(e);
  }
  {
    Entry e;
    e.fast = false;
    e.vec = 1;
    e.k = wide_carry ? 16 : 32;
    e.wpb = wide_carry ? 16 : 8;
    e.threads = 64 * e.wpb;
    e.blocks_per_cu = wide_carry ? 1 : 3;
    e.symbol = L.name + "_s";
    src << "extern \"C\" __global__ void __launch_bounds__(" << e.threads << ") " << e.symbol << "(const " << T
        << "* in, " << T << "* out, long long rows, long long cols, unsigned long long* status, "
        << "unsigned* counter, unsigned ticket_base, unsigned epoch, unp::waits wt) {\n  unp::scan_lookback<" << T << ", " << f.op0
        << ", " << (f.exclusive ? "true" : "false") << ", " << (f.reverse ? "true" : "false") << ", 1, " << e.k
        << ", " << e.wpb << ", " << kScanStatusWords << (fixed ? ", true" : "")
        << ">(in, out, rows, cols, status, counter, ticket_base, epoch, wt);\n}\n";
    L.entries.push_back(e);
  }
  src << scan_strided_entry(f, L);
  L.threads = L.entries[0].threads;
  L.blocks_per_cu = 1;
  L.source = src.str();
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"scan\",\"dtype\":\"" << kind_name(f.dtype)
    << "\",\"op\":\"" << op_name(f.op0) << "\",\"exclusive\":" << (f.exclusive ? "true" : "false")
    << ",\"reverse\":" << (f.reverse ? "true" : "false") << ",\"rank\":" << f.rank
    << ",\"schedule\":\"" << (fixed ? "fixed" : "device") << "\""
    << ",\"params\":[{\"name\":\"in0\",\"kind\":\"buffer\",\"role\":\"Read\"},{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\"}";
  for (int d = 0; d < f.rank; ++d) j << ",{\"name\":\"n" << d << "\",\"kind\":\"scalar\",\"dtype\":\"I32\"}";
  j << "],\"launch\":{\"block\":[" << L.threads << ",1,1],\"grid\":\"cu_count*" << L.blocks_per_cu
    << "\",\"grid_policy\":\"persistent blocks draw one block-tile ticket per round\"},\"entries\":[";
  for (size_t i = 0; i < L.entries.size(); ++i)
    j << (i ? "," : "") << "{\"symbol\":\"" << L.entries[i].symbol << "\",\"vec\":" << L.entries[i].vec
      << ",\"k\":" << L.entries[i].k << ",\"waves\":" << L.entries[i].wpb
      << ",\"block\":" << L.entries[i].threads << ",\"blocks_per_cu\":" << L.entries[i].blocks_per_cu
      << ",\"block_tile\":" << 64 * L.entries[i].vec * L.entries[i].k * L.entries[i].wpb << ",\"when\":\""
      << (L.entries[i].strided ? kStridedWhen
          : L.entries[i].fast  ? "scanned extent % vec == 0 and in0/out 16-byte aligned"
                               : "otherwise")
      << "\"}";
  j << "],\"workspace\":{\"status\":\"tiles * " << kScanStatusWords * 8
    << " bytes, zeroed once\",\"counter\":4,\"stall\":4,\"host_state\":[\"epoch\",\"ticket_base\"]}"
    << ",\"compiler_args\":[\"--offload-arch=gfx950\",\"-O3\",\"-Xclang\",\"-target-feature\",\"-Xclang\",\"-packed-fp32-ops\"]"
    << ",\"fidelity_notes\":["
    << json_str(fixed
                    ? "fixed schedule: a tile's carry is G(k-1) folded with the wave-tree prefix of its group's earlier tile "
                      "aggregates (groups of 64 tiles per row, G(k) = G(k-1) folded with the group's wave-tree total), an "
                      "association the tile size alone fixes: the same bits on every launch and any grid for one entry. "
                      "The entry follows from the row length and the buffers' alignment: rows of whole 16-byte vectors at "
                      "16-byte-aligned addresses take the staged entry (18432-element tiles), others the register entry "
                      "(16384-element tiles), whose bits may differ; a strided view runs the serial order. Float Sum / "
                      "Mean fold in f64 within the declared per-prefix bound gamma_(n-1)*sum|x| + 1/2 ulp; Max/Min keep one "
                      "NaN payload and zero sign launch to launch"
                : kind_is_float(f.dtype) && (f.op0 == UNP_OP_SUM || f.op0 == UNP_OP_MEAN)
                    ? "float Sum / Mean: every prefix is an f64 fold of the same elements in a different order (tile-local "
                      "striped scan plus decoupled look-back; a Mean divides it by the count once); within the declared "
                      "per-prefix bound gamma_(n-1)*sum|x| + 1/2 ulp; bit-equal whenever the f64 partial sums are exact. "
                      "Not reproducible run to run: the carry's association depends on how many tiles each look-back "
                      "folded before it met an inclusive prefix, which depends on timing; every launch is within the bound"
                    : "order-independent fold: bit-exact against the serial scan except NaN payload and the sign of a zero in Max/Min")
    << "," << json_str("one single-pass decoupled look-back launch replaces the KernelFn's block-per-row three-phase schedule")
    << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

static int32_t lower_gather(const unp_form& f, Lowered& L, std::string& why) {
  if (f.rank < 1 || f.rank > 8) {
    why = "a rank-0 gather has no loop";
    return UNP_LIFT_DECLINE;
  }
  const size_t eb = kind_bytes(f.dtype);
  if (eb == 0) {
    why = "a gather of a sub-byte or unknown element kind";
    return UNP_UNSUPPORTED_DTYPE;
  }
  if (f.index_dtype != UNP_I32 && f.index_dtype != UNP_I64 && f.index_dtype != UNP_U32) {
    why = "a non-integer gather index";
    return UNP_LIFT_DECLINE;
  }
  if (!oob_name(f.oob)) {
    why = "an unknown out-of-range policy";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (f.data_slot != 0 && f.data_slot != 1) {
    why = "an ill-formed gather";
    return UNP_LIFT_DECLINE;
  }
  // The gathered axis: axes_mask's one bit, or axis 0 (the row gather of an embedding).
  int32_t axis = 0;
  if (f.axes_mask) {
    if ((f.axes_mask & (f.axes_mask - 1)) != 0 || (f.axes_mask >> f.rank) != 0) {
      why = "a gather gathers exactly one axis inside the rank";
      return UNP_LIFT_DECLINE;
    }
    axis = __builtin_ctz(f.axes_mask);
  }
  L.scan_axis = axis;  // the gathered axis (the executor sees the output as A x NI rows)
  const bool batch = axis > 0;
  const char* I = ctype(f.index_dtype);
  std::ostringstream name;
  name << "unp_gather_" << (batch ? "select_" : "rows_") << lower_name(f.dtype) << "_by_" << lower_name(f.index_dtype)
       << "_" << oob_name(f.oob);
  L.name = name.str();
  L.threads = 256;
  L.blocks_per_cu = 1;
  std::ostringstream src;
  src << header(L.name, f);
  const int units[2] = {16, (int)eb};
  for (int i = 0; i < 2; ++i) {
    if (i == 1 && units[1] == 16) break;
    Entry e;
    e.fast = (i == 0);
    e.vec = units[i];
    e.symbol = L.name + (i == 0 ? "_u16" : "_u" + std::to_string(units[i]));
    // 16-byte units: one wave per block and two blocks per CU, two 8 KiB rows of a wave in
    // flight (measured best at cfg4's 65536 x 8 KiB); narrower units: four waves per block.
    const int U = units[i] == 16 ? 8 : 16;
    e.threads = units[i] == 16 ? 64 : 256;
    e.blocks_per_cu = units[i] == 16 ? 2 : 1;
    src << "extern \"C\" __global__ void __launch_bounds__(" << e.threads << ") " << e.symbol
        << "(const unsigned char* table, const " << I << "* ids, unsigned char* out, long long n_rows, "
        << "long long row_bytes, " << I << " src_extent" << (batch ? ", long long ni" : "")
        << ") {\n  unp::gather_rows<" << I << ", " << f.oob << ", " << units[i] << ", " << e.threads << ", " << U
        << ", 2" << (batch ? ", true" : "") << ">(table, ids, out, n_rows, row_bytes, src_extent"
        << (batch ? ", ni" : "") << ");\n}\n";
    L.entries.push_back(e);
  }
  {
    // Storage images that are not the dense layout above: one lane per output element, the table,
    // index and output addressed through their strides, the element moved as raw bits.
    Entry e;
    e.strided = true;
    e.vec = (int)eb;
    e.threads = 256;
    e.blocks_per_cu = 8;
    e.symbol = L.name + "_x";
    const char* E = eb == 1 ? "unsigned char" : eb == 2 ? "unsigned short" : eb == 4 ? "unsigned int" : "unsigned long long";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(const " << E << "* table, const "
        << I << "* ids, " << E << "* out, unp::gather_view v, " << I << " src_extent) {\n  unp::gather_strided<" << E
        << ", " << I << ", " << f.oob << ">(table, ids, out, v, src_extent);\n}\n";
    L.entries.push_back(e);
  }
  L.source = src.str();
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"gather\",\"dtype\":\"" << kind_name(f.dtype)
    << "\",\"index_dtype\":\"" << kind_name(f.index_dtype) << "\",\"oob\":\"" << oob_name(f.oob)
    << "\",\"axis\":" << axis << ",\"rank\":" << f.rank << ",\"params\":[{\"name\":\"in0\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\""
    << kind_name(f.data_slot == 0 ? f.dtype : f.index_dtype) << "\"},{\"name\":\"in1\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\""
    << kind_name(f.data_slot == 1 ? f.dtype : f.index_dtype)
    << "\"},{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\"}";
  for (int d = 0; d < f.rank; ++d) j << ",{\"name\":\"n" << d << "\",\"kind\":\"scalar\",\"dtype\":\"I32\"}";
  j << ",{\"name\":\"src_extent\",\"kind\":\"scalar\",\"dtype\":\"" << kind_name(f.index_dtype)
    << "\"}],\"launch\":{\"block\":[" << L.entries[0].threads << ",1,1],\"grid\":\"cu_count*"
    << L.entries[0].blocks_per_cu
    << "\",\"grid_policy\":\"waves stride over output rows (the output seen as A x NI rows of the axes after the "
       "gathered one, the index 1-D over NI); whole rows of 64 x 8 units two at a time per wave\"},\"entries\":[";
  for (size_t i = 0; i < L.entries.size(); ++i)
    j << (i ? "," : "") << "{\"symbol\":\"" << L.entries[i].symbol << "\",\"unit_bytes\":" << L.entries[i].vec
      << ",\"when\":\""
      << (L.entries[i].strided ? kStridedWhen
          : L.entries[i].fast  ? "row bytes % 16 == 0 and table/out 16-byte aligned"
                               : "otherwise")
      << "\"}";
  j << "],\"workspace\":null,\"fidelity_notes\":[" << json_str("a raw bit move: bit-exact for every grid and block")
    << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

static int32_t lower_dequant(const unp_form& f, Lowered& L, std::string& why) {
  if (f.q_kind != UNP_U4 && f.q_kind != UNP_I4) {
    why = "dequant weights must be U4 or I4";
    return UNP_UNSUPPORTED_DTYPE;
  }
  if (f.z_kind != UNP_U4 && f.z_kind != UNP_I4) {
    why = "dequant zero points must be U4 or I4";
    return UNP_UNSUPPORTED_DTYPE;
  }
  if (f.out_kind != UNP_BF16) {
    why = "dequant output other than Bf16";
    return UNP_UNSUPPORTED_DTYPE;
  }
  if (f.group < 1) {
    why = "a dequant group of zero columns";
    return UNP_UNSUPPORTED_KERNEL;
  }
  const bool qs = f.q_kind == UNP_I4, zs = f.z_kind == UNP_I4;
  std::ostringstream name;
  name << "unp_dequant_" << lower_name(f.q_kind) << "_z" << lower_name(f.z_kind) << "_g" << f.group << "_bf16";
  L.name = name.str();
  // Two blocks of four waves per CU, each wave with a tile of 4 x 64 items (1 KiB of q,
  // 4 KiB of bf16) and the next tile's loads in flight: measured best at 8192 x 28672.
  L.threads = 256;
  L.blocks_per_cu = 2;
  std::ostringstream src;
  src << header(L.name, f);
  const char* sig =
      "(const unsigned char* q, const unsigned short* scale, const unsigned char* zero, unsigned short* out, "
      "long long rows, long long cols)";
  if (f.group % 8 == 0) {
    Entry e;
    e.fast = true;
    e.vec = 8;
    e.symbol = L.name + "_v";
    src << "extern \"C\" __global__ void " << kLaunchBounds << " " << e.symbol << sig << " {\n  unp::dequant4_bf16<"
        << (qs ? "true" : "false") << ", " << (zs ? "true" : "false") << ", " << f.group
        << ", 256, 4>(q, scale, zero, out, rows, cols);\n}\n";
    L.entries.push_back(e);
  }
  {
    Entry e;
    e.fast = false;
    e.vec = 1;
    e.symbol = L.name + "_s";
    src << "extern \"C\" __global__ void " << kLaunchBounds << " " << e.symbol << sig << " {\n  unp::dequant4_bf16_any<"
        << (qs ? "true" : "false") << ", " << (zs ? "true" : "false") << ", " << f.group
        << ", 256>(q, scale, zero, out, rows, cols);\n}\n";
    L.entries.push_back(e);
  }
  L.source = src.str();
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"dequant4\",\"q\":\"" << kind_name(f.q_kind)
    << "\",\"zero\":\"" << kind_name(f.z_kind) << "\",\"scale\":\"F16\",\"out\":\"Bf16\",\"group\":" << f.group
    << ",\"params\":[{\"name\":\"w\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\"" << kind_name(f.q_kind)
    << "\"},{\"name\":\"scale\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\"F16\"},{\"name\":\"zero\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\""
    << kind_name(f.z_kind)
    << "\"},{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\",\"dtype\":\"Bf16\"},{\"name\":\"n0\",\"kind\":\"scalar\",\"dtype\":\"I32\"},{\"name\":\"n1\",\"kind\":\"scalar\",\"dtype\":\"I32\"}]"
    << ",\"launch\":{\"block\":[256,1,1],\"grid\":\"cu_count*" << L.blocks_per_cu
    << "\",\"grid_policy\":\"waves take 256 consecutive 8-element items per step, the next step loaded ahead, and stride over the grid\"},\"entries\":[";
  for (size_t i = 0; i < L.entries.size(); ++i)
    j << (i ? "," : "") << "{\"symbol\":\"" << L.entries[i].symbol << "\",\"when\":\""
      << (L.entries[i].fast ? "cols % group == 0, w 4-byte and out 16-byte aligned" : "otherwise") << "\"}";
  j << "],\"workspace\":null,\"fidelity_notes\":["
    << json_str("exact integer difference and exact f32 product; one round-to-nearest-even to bf16: bit-exact")
    << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

// The dequantizing GEMM: the int8 MFMA entry when the group holds whole 32-deep MFMA steps, and
// a serial entry for any other shape.  KC, the k-values staged in LDS per chunk, is the largest
// multiple of 32 that divides the group within 512 bytes of an I8 column or 128 of an I32's.
static int32_t lower_dequant_gemm(const unp_form& f, Lowered& L, std::string& why) {
  if (f.q_kind != UNP_U4 && f.q_kind != UNP_I4) {
    why = "dequant-GEMM weights must be U4 or I4";
    return UNP_UNSUPPORTED_DTYPE;
  }
  if (f.dtype != UNP_I8 && f.dtype != UNP_I32) {
    why = "dequant-GEMM activations must be I8 or I32";
    return UNP_UNSUPPORTED_DTYPE;
  }
  if (f.group < 1) {
    why = "a dequant group of zero columns";
    return UNP_UNSUPPORTED_KERNEL;
  }
  const bool qs = f.q_kind == UNP_I4;
  const int xb = f.dtype == UNP_I32 ? 4 : 1;
  const char* xt = xb == 4 ? "int" : "signed char";
  int kc = 0;
  for (int c = 32; c <= (xb == 4 ? 128 : 512); c += 32)
    if (f.group % c == 0) kc = c;
  // The streaming schedule: groups of whole 64-value chunks.  Stage chunk 128 (I8, when it
  // divides the group) or 64.  I8 with 128-value chunks: 2 x 2 waves, each with 2 x 2 tiles of
  // 32 x 32 (128 x 128 per block); I32: four waves stacked over 128 rows with 1 x 2 tiles each
  // (128 x 64); both with three stages and two blocks per CU.  I8 with 64-value chunks: four
  // waves of one tile (128 x 32), four stages.
  const int skc = f.group % 64 != 0 ? 0 : (xb == 1 && f.group % 128 == 0 ? 128 : 64);
  const bool big = xb == 1 && skc == 128, two = big || xb == 4;
  const int swr = big ? 2 : 4, swc = big ? 2 : 1, stm = big ? 2 : 1, stn = two ? 2 : 1, sns = two ? 3 : 4;
  // The decode schedule (up to 64 columns for I8, 128 for I32): groups of 1..4 whole 128-value steps (1..2 for I32
  // activations, whose four digit planes take four times the x' bytes).  Two m-tiles per wave; I8
  // with 1, 2 or 4 column tiles of 16 sharing each unpacked w operand, two steps in flight (or one
  // group); I32 with one column tile and two steps in flight.
  const int spg = f.group % 128 == 0 ? f.group / 128 : 0;
  const bool dec = spg >= 1 && spg <= (xb == 1 ? 4 : 2);
  const int dmt = 2, dd = xb == 1 ? (spg <= 1 ? 2 : spg) : spg, dmaxg = 32;
  std::ostringstream name;
  name << "unp_dequant_gemm_" << lower_name(f.q_kind) << "_g" << f.group << "_" << lower_name(f.dtype) << "_i32";
  L.name = name.str();
  L.threads = 256;
  L.blocks_per_cu = 8;
  std::ostringstream src;
  src << header(L.name, f);
  const std::string sig = std::string("(const unsigned char* w, const int* zero, const int* scale, const ") + xt +
                          "* x, int* out, long long R, long long K, long long C)";
  // Decode entries: eight waves of 32 rows per block (256 rows), one block per CU, the block's x'
  // staged in LDS.  I8 with one column tile holds its split's every step (at most 32 steps);
  // the others stream x' through two LDS buffers of P steps, 16 KiB each (P a multiple of the
  // steps in flight), one phase ahead.
  auto dec_entry = [&](const char* suffix, int nc, int xm, int maxg) {
    const int xs = nc * xb * 2048, dd2 = xb == 1 ? dd : 2;
    const int P = xm == 1 ? 0 : std::max(dd2, 16384 / xs / dd2 * dd2);
    Entry e;
    e.fast = true;
    e.symbol = L.name + suffix;
    e.vec = 16 * dmt * 8;  // rows per block
    e.cols = 16 * nc;      // columns per block
    e.k = maxg;            // groups per split at most
    e.threads = 512;
    e.blocks_per_cu = 1;
    src << "extern \"C\" __global__ void __launch_bounds__(512) " << e.symbol
        << "(const unsigned char* w, const int* zero, const int* scale, const unsigned char* xp, const unsigned* xsum, "
           "int* out, long long R, long long K, long long C, long long Cp, long long S) {\n  unp::dqg_dec<"
        << (qs ? "true" : "false") << ", " << xb << ", " << f.group << ", " << dmt << ", " << nc << ", " << dd2 << ", "
        << maxg << ", 8, " << xm << ", " << P << ">(w, zero, scale, xp, xsum, out, R, K, C, Cp, S);\n}\n";
    L.entries.push_back(e);
  };
  if (dec && xb == 1) {
    dec_entry("_dec1x", 1, 1, 32 / spg);
    dec_entry("_dec2", 2, 2, dmaxg);
    dec_entry("_dec4", 4, 2, dmaxg);
  } else if (dec) {
    // 56 groups per split (the scales then fill 114 KiB of LDS): at 8192 rows, 4 splits make whole
    // rounds of 256 blocks for 32, 64 and 128 columns, where 32 groups need 7.
    dec_entry("_dec1", 1, 2, 56);
  }
  if (skc) {
    Entry e;
    e.fast = true;
    e.symbol = L.name + "_stream";
    e.blocks_per_cu = 2;
    e.vec = 32 * swr * stm;  // rows per block
    e.k = 32 * swc * stn;    // columns per block
    src << "extern \"C\" __global__ void __launch_bounds__(256" << (two ? ", 2" : "") << ") " << e.symbol
        << "(const unsigned char* w, const int* zero, const int* scale, const unsigned char* xp, const unsigned* xsum, "
           "int* out, long long R, long long K, long long C, long long Cp, long long S) {\n  unp::dqg_stream<"
        << (qs ? "true" : "false") << ", " << xb << ", " << f.group << ", " << skc << ", " << swr << ", " << swc
        << ", " << stm << ", " << stn << ", " << sns << ">(w, zero, scale, xp, xsum, out, R, K, C, Cp, S);\n}\n";
    L.entries.push_back(e);
  }
  if (kc) {
    Entry e;
    e.fast = true;
    e.symbol = L.name + "_mfma";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << sig << " {\n  unp::dqgemm_mfma<"
        << (qs ? "true" : "false") << ", " << xb << ", " << f.group << ", " << kc
        << ">(w, zero, scale, x, out, R, K, C);\n}\n";
    L.entries.push_back(e);
  }
  {
    Entry e;
    e.fast = false;
    e.symbol = L.name + "_any";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << sig << " {\n  unp::dqgemm_any<"
        << (qs ? "true" : "false") << ", " << xt << ", 256>(w, zero, scale, x, out, R, K, C, " << f.group
        << ");\n}\n";
    L.entries.push_back(e);
  }
  if (skc) {
    Entry e;
    e.fast = false;
    e.symbol = L.name + "_prep";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(const " << xt
        << "* x, unsigned char* xp, unsigned* xsum, long long K, long long C, long long Cp, long long G, int* out, "
           "long long n_out) {\n  unp::dqg_prep<"
        << xt << ", " << xb << ", " << skc << ">(x, xp, xsum, K, C, Cp, G, out, n_out);\n}\n";
    L.entries.push_back(e);
  }
  if (dec) {
    Entry e;
    e.fast = false;
    e.symbol = L.name + "_prep16";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(const " << xt
        << "* x, unsigned char* xp, unsigned* xsum, long long K, long long C, long long Cp, long long G, int* out, "
           "long long n_out) {\n  unp::dqg_prep16<"
        << xt << ", " << xb << ">(x, xp, xsum, K, C, Cp, G, out, n_out);\n}\n";
    L.entries.push_back(e);
  }
  L.source = src.str();
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"dequant_gemm\",\"w\":\"" << kind_name(f.q_kind)
    << "\",\"zero\":\"I32\",\"scale\":\"I32\",\"x\":\"" << kind_name(f.dtype) << "\",\"out\":\"I32\",\"group\":"
    << f.group << ",\"chunk\":" << kc << ",\"stream_chunk\":" << skc << ",\"decode_steps\":" << (dec ? (xb == 1 ? dd : 2) : 0)
    << ",\"params\":[{\"name\":\"w\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\"" << kind_name(f.q_kind)
    << "\"},{\"name\":\"zero\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\"I32\"},{\"name\":\"scale\",\"kind\":"
       "\"buffer\",\"role\":\"Read\",\"dtype\":\"I32\"},{\"name\":\"x\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\""
    << kind_name(f.dtype)
    << "\"},{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\",\"dtype\":\"I32\"}"
    << ",{\"name\":\"n0\",\"kind\":\"scalar\",\"dtype\":\"I32\"},{\"name\":\"n1\",\"kind\":\"scalar\",\"dtype\":\"I32\"},{"
       "\"name\":\"n2\",\"kind\":\"scalar\",\"dtype\":\"I32\"}]"
    << ",\"launch\":{\"block\":[256,1,1],\"grid_policy\":\"device-class grids whose blocks stride over items. dec: "
       "a prep launch (cu_count*8 blocks) over (group, 16 columns), then cu_count blocks of 512 threads over "
       "(row tiles rounded up to 8) x splits x column tiles items of 256 rows x 16, 32 or 64 columns (I8) or x 16 "
       "(I32), the split's x' in LDS (whole for one I8 column tile, else streamed through two buffers), a split's "
       "groups at most 32 (56 for I32), the splits adding into out with atomics; stream: a prep launch over "
       "(group, 64 columns), then cu_count*2 blocks over (row tiles x splits, rounded up to 8) x column tiles items "
       "of 128 x 128 (I8, 128-value chunks), 128 x 64 (I32) or 128 x 32 outputs, the splits adding into out with "
       "atomics; mfma: cu_count*4 blocks over 64 x 64 output tiles; any: threads stride over the outputs\"},\"entries\":[";
  for (size_t i = 0; i < L.entries.size(); ++i) {
    const std::string& sym = L.entries[i].symbol;
    const bool is_stream = sym.size() > 7 && sym.compare(sym.size() - 7, 7, "_stream") == 0;
    const bool is_prep = sym.size() > 5 && sym.compare(sym.size() - 5, 5, "_prep") == 0;
    const bool is_dec = L.entries[i].cols > 0;
    const bool is_prep16 = sym.size() > 7 && sym.compare(sym.size() - 7, 7, "_prep16") == 0;
    j << (i ? "," : "") << "{\"symbol\":\"" << sym << "\",\"when\":\""
      << (is_dec ? "C <= 64 for I8, C <= 128 for I32 (the entry whose column tiles cover C, or the widest), "
                   "K % group == 0, w 16-byte aligned, "
                   "w and repacked x under 2 GiB; after the prep16 launch (buffer loads into VGPRs, "
                   "v_mfma_i32_16x16x64_i8)"
          : is_prep16 ? "before the dec entry: x repacked for 16-column tiles, group column sums, out zeroed"
          : is_stream ? "K % group == 0, w 16-byte aligned, scales and column sums under 2 GiB; after the prep "
                      "launch (LDS-staged DMA, v_mfma_i32_32x32x32_i8, the zero-point term on the MFMA in "
                      "byte digits after the loop)"
                    : is_prep ? "before the stream entry: x repacked into digit planes and group column sums"
                              : L.entries[i].fast ? "K % group == 0, C % 4 == 0, x aligned to 4 elements, w to 8 "
                                                    "bytes (v_mfma_i32_32x32x32_i8)"
                                                  : "otherwise")
      << "\"}";
  }
  j << "],\"workspace\":" << (skc ? "\"dec and stream: K x Cp x planes bytes of repacked x, then (K / group x Cp + 64) "
                                    "u32 column sums (Cp = C rounded up to the entry's columns per block, at least 64 for stream)\""
                                  : "null")
    << ",\"compiler_args\":[\"--offload-arch=gfx950\",\"-O3\",\"-Xclang\",\"-target-feature\",\"-Xclang\",\"-packed-fp32-ops\"]"
    << ",\"fidelity_notes\":["
    << json_str("I32 arithmetic that wraps, regrouped in that ring as sum_g scale * (sum_k w * x - zero * sum_k x); "
                "the sums of w * x run on the int8 MFMA, I32 activations as four signed byte digits: bit-exact "
                "against the serial kernel for every input")
    << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

// ---- Access::RowReduce ---------------------------------------------------------------------

namespace {

// A ScalarExpr over Input(k) / Reduced(t) leaves as a C++ double expression (f64 evaluation,
// the caller rounds once).  False, with the node named in `why`, outside the vocabulary this
// backend spells.
// `reuse`, when set, is a subtree whose value the caller already holds: every node equal to it
// is spelled `c` instead.
bool expr_cpp(const kir::J& e, const char* T, std::string& out, std::string& why, const kir::J* reuse = nullptr) {
  using kir::J;
  if (reuse && e == *reuse) {
    out = "c";
    return true;
  }
  if (e.t != J::Obj || e.o.size() != 1) {
    why = "a malformed ScalarExpr";
    return false;
  }
  const std::string& tag = e.o[0].first;
  const J& p = e.o[0].second;
  auto sub = [&](size_t i, std::string& o) {
    return p.t == J::Arr && i < p.a.size() && expr_cpp(p.a[i], T, o, why, reuse);
  };
  if (tag == "Input" || tag == "Reduced") {
    if (!p.is_int || p.i < 0) {
      why = "a malformed leaf";
      return false;
    }
    out = std::string(tag == "Input" ? "x[" : "r[") + std::to_string(p.i) + "]";
    return true;
  }
  if (tag == "Const") {
    if (p.t == J::Str) {
      if (p.s == "NaN") out = "__builtin_nan(\"\")";
      else if (p.s == "inf") out = "__builtin_inf()";
      else if (p.s == "-inf") out = "(-__builtin_inf())";
      else {
        why = "a Const tag `" + p.s + "`";
        return false;
      }
      return true;
    }
    if (p.t != J::Num) {
      why = "a malformed Const";
      return false;
    }
    char buf[64];
    std::snprintf(buf, sizeof buf, "%a", p.d);  // exact: a hexadecimal floating literal
    out = std::string("(") + buf + ")";
    return true;
  }
  std::string a, b, c;
  if (tag == "Add" || tag == "Sub" || tag == "Mul" || tag == "Div") {
    if (!sub(0, a) || !sub(1, b)) return false;
    const char* o = tag == "Add" ? " + " : tag == "Sub" ? " - " : tag == "Mul" ? " * " : " / ";
    out = "(" + a + o + b + ")";
    return true;
  }
  if (tag == "Fma" || tag == "Select") {
    if (!sub(0, a) || !sub(1, b) || !sub(2, c)) return false;
    out = (tag == "Fma" ? "fma(" : "unp::xf::select(") + a + ", " + b + ", " + c + ")";
    return true;
  }
  if (tag == "Unary") {
    if (p.t != J::Arr || p.a.size() != 2 || p.a[0].t != J::Str || !sub(1, a)) {
      if (why.empty()) why = "a malformed Unary";
      return false;
    }
    static const struct {
      const char* op;
      const char* fn;
    } un[] = {{"Abs", "fabs"},         {"Sqr", "unp::xf::sqr"},   {"Sqrt", "sqrt"},
              {"Rsqrt", "unp::xf::rsqrt"}, {"Recip", "unp::xf::recip"}, {"Exp", "exp"},
              {"Log", "log"},          {"Tanh", "tanh"},          {"Sigmoid", "unp::xf::sigmoid"},
              {"Relu", "unp::xf::relu"}, {"Erf", "erf"},           {"Gelu", "unp::xf::gelu"},
              {"Silu", "unp::xf::silu"}, {"Sin", "sin"},           {"Cos", "cos"},
              {"Floor", "floor"},      {"Ceil", "ceil"},          {"Round", "rint"},
              {"Erfc", "erfc"},        {"Trunc", "trunc"},        {"Exp2", "exp2"},
              {"Expm1", "expm1"},      {"Log2", "log2"},          {"Log10", "log10"},
              {"Log1p", "log1p"},      {"Sinh", "sinh"},          {"Cosh", "cosh"},
              {"Tan", "tan"},          {"Asin", "asin"},          {"Acos", "acos"},
              {"Atan", "atan"},        {"Asinh", "asinh"},        {"Acosh", "acosh"},
              {"Atanh", "unp::xf::atanh_odd"}, {"Cbrt", "cbrt"}};
    const std::string& op = p.a[0].s;
    if (op == "Neg") {
      out = "(-" + a + ")";
      return true;
    }
    if (op == "Sign" || op == "Step") {
      out = std::string("unp::xf::") + (op == "Sign" ? "sign<" : "step<") + T + ">(" + a + ")";
      return true;
    }
    for (const auto& u : un)
      if (op == u.op) {
        out = std::string(u.fn) + "(" + a + ")";
        return true;
      }
    why = "the unary op " + op;
    return false;
  }
  if (tag == "Binary") {
    if (p.t != J::Arr || p.a.size() != 3 || p.a[0].t != J::Str || !sub(1, a) || !sub(2, b)) {
      if (why.empty()) why = "a malformed Binary";
      return false;
    }
    const std::string& op = p.a[0].s;
    static const struct {
      const char* op;
      const char* fn;
    } bn[] = {{"Max", "unp::xf::max_prop"}, {"Min", "unp::xf::min_prop"}, {"Pow", "pow"},
              {"Rem", "unp::xf::rem_floor"}, {"RemTrunc", "fmod"},         {"Atan2", "atan2"},
              {"Copysign", "copysign"},     {"FmaxIeee", "fmax"},         {"FminIeee", "fmin"}};
    for (const auto& u : bn)
      if (op == u.op) {
        out = std::string(u.fn) + "(" + a + ", " + b + ")";
        return true;
      }
    static const struct {
      const char* op;
      const char* c;
    } cmp[] = {{"CmpEq", "=="}, {"CmpNe", "!="}, {"CmpLt", "<"}, {"CmpLe", "<="}, {"CmpGt", ">"}, {"CmpGe", ">="}};
    for (const auto& u : cmp)
      if (op == u.op) {
        out = "((" + a + " " + u.c + " " + b + ") ? 1.0 : 0.0)";
        return true;
      }
    why = "the binary op " + op;
    return false;
  }
  why = "the expression node " + tag;
  return false;
}

// ---- integer expressions (oracle/kernel_eval.rs:809-848, 1114-1175) ---------------------------

// The C++ type of an integer compute kind this backend spells expressions at.
const char* int_ctype(int32_t kind) {
  switch (kind) {
    case UNP_I32: return "int";
    case UNP_I64: return "long long";
    case UNP_U32: return "unsigned int";
    case UNP_U64: return "unsigned long long";
    default: return nullptr;
  }
}

// The type of an expression node under an integer compute dtype (types.rs:679-751 for the nodes
// the integer evaluator takes): an Input is the compute dtype, a ConstInt its own kind, a Cast its
// target, arithmetic its operands' common type, a comparison the compute dtype's 0/1, a Select its
// arms'.  -1 for a node outside that subset or operands of different types.
int32_t int_node_type(const kir::J& e, int32_t compute) {
  using kir::J;
  if (e.t != J::Obj || e.o.size() != 1) return -1;
  const std::string& tag = e.o[0].first;
  const J& p = e.o[0].second;
  if (tag == "Input") return compute;
  if (tag == "ConstInt") return p.t == J::Arr && p.a.size() == 2 && p.a[1].t == J::Str ? kind_from_name(p.a[1].s) : -1;
  if (tag == "Cast") {
    const J* to = p.t == J::Arr && p.a.size() == 2 ? p.a[1].get("to") : nullptr;
    return to && to->t == J::Str ? kind_from_name(to->s) : -1;
  }
  auto same = [&](const J& a, const J& b) {
    const int32_t x = int_node_type(a, compute), y = int_node_type(b, compute);
    return x == y ? x : -1;
  };
  if (tag == "Add" || tag == "Sub" || tag == "Mul" || tag == "Div")
    return p.t == J::Arr && p.a.size() == 2 ? same(p.a[0], p.a[1]) : -1;
  if (tag == "Binary") {
    if (p.t != J::Arr || p.a.size() != 3 || p.a[0].t != J::Str) return -1;
    const int32_t t = same(p.a[1], p.a[2]);
    return t >= 0 && p.a[0].s.compare(0, 3, "Cmp") == 0 ? compute : t;
  }
  if (tag == "Select") return p.t == J::Arr && p.a.size() == 3 ? same(p.a[1], p.a[2]) : -1;
  return -1;
}

// An integer expression spelled at the integer kind `t` as the reference's kernel evaluator
// computes it (eval_int, kernel_eval.rs:809-848): every operand at `t` except a Cast's operand, a
// comparison's operands and a Select's condition, which are read at their own type.  The total
// rule of docs/int-div-shift-semantics.md (rules 1-3) is in the device library's unp::xi helpers:
// Add/Sub/Mul wrap, a zero divisor and signed MIN / -1 give the dividend, shift counts are taken
// modulo the width.  A ConstInt is its value wrapped to `t` (kernel_eval.rs:1165-1174).
bool int_expr_cpp(const kir::J& e, int32_t t, int32_t compute, std::string& out, std::string& why) {
  using kir::J;
  const char* T = int_ctype(t);
  if (!T) {
    why = std::string("an integer expression at ") + (kind_name(t) ? kind_name(t) : "an unknown kind");
    return false;
  }
  if (e.t != J::Obj || e.o.size() != 1) {
    why = "a malformed ScalarExpr";
    return false;
  }
  const std::string& tag = e.o[0].first;
  const J& p = e.o[0].second;
  auto at = [&](const J& x, int32_t ty, std::string& o) { return int_expr_cpp(x, ty, compute, o, why); };
  auto own = [&](const J& x, std::string& o) {
    const int32_t ty = int_node_type(x, compute);
    if (!int_ctype(ty)) {
      if (why.empty()) why = "an operand outside the integer kinds I32, I64, U32 and U64";
      return false;
    }
    return at(x, ty, o);
  };
  if (tag == "Input") {
    if (!p.is_int || p.i < 0 || t != compute) {
      why = "a malformed Input";
      return false;
    }
    out = "x[" + std::to_string(p.i) + "]";
    return true;
  }
  if (tag == "ConstInt") {
    if (p.t != J::Arr || p.a.size() != 2 || !p.a[0].is_int) {
      why = "a ConstInt outside the 64-bit signed range";
      return false;
    }
    const int64_t v = p.a[0].i;
    char buf[64];
    if (t == UNP_I32) std::snprintf(buf, sizeof buf, "(int)(%d)", (int)(int32_t)(uint32_t)(uint64_t)v);
    else if (t == UNP_U32) std::snprintf(buf, sizeof buf, "(unsigned int)%uu", (unsigned)(uint32_t)(uint64_t)v);
    else if (t == UNP_U64) std::snprintf(buf, sizeof buf, "(unsigned long long)%lluull", (unsigned long long)(uint64_t)v);
    else if (v == INT64_MIN) std::snprintf(buf, sizeof buf, "(-9223372036854775807ll - 1ll)");
    else std::snprintf(buf, sizeof buf, "(long long)(%lldll)", (long long)v);
    out = buf;
    return true;
  }
  if (tag == "Cast") {
    // An integer-to-integer wrap to `t` (a Cast to another type is a mixed expression).
    const J* sat = p.t == J::Arr && p.a.size() == 2 ? p.a[1].get("sat") : nullptr;
    if (int_node_type(e, compute) != t || !sat || sat->t != J::Str || sat->s != "Wrap") {
      why = "a Cast other than an integer wrap to the expression's type";
      return false;
    }
    std::string a;
    if (!own(p.a[0], a)) return false;
    out = "(" + std::string(T) + ")(" + a + ")";
    return true;
  }
  std::string a, b, c;
  if (tag == "Add" || tag == "Sub" || tag == "Mul" || tag == "Div") {
    if (p.t != J::Arr || p.a.size() != 2 || !at(p.a[0], t, a) || !at(p.a[1], t, b)) return false;
    std::string fn = tag == "Add" ? "add" : tag == "Sub" ? "sub" : tag == "Mul" ? "mul" : "div";
    out = "unp::xi::" + fn + "<" + T + ">(" + a + ", " + b + ")";
    return true;
  }
  if (tag == "Binary") {
    if (p.t != J::Arr || p.a.size() != 3 || p.a[0].t != J::Str) {
      why = "a malformed Binary";
      return false;
    }
    const std::string& op = p.a[0].s;
    static const struct {
      const char* op;
      const char* fn;
    } ib[] = {{"Shl", "shl"}, {"Shr", "shr"}, {"Min", "min"}, {"Max", "max"},
              {"BitAnd", "bit_and"}, {"BitOr", "bit_or"}, {"BitXor", "bit_xor"}};
    for (const auto& u : ib)
      if (op == u.op) {
        if (!at(p.a[1], t, a) || !at(p.a[2], t, b)) return false;
        out = std::string("unp::xi::") + u.fn + "<" + T + ">(" + a + ", " + b + ")";
        return true;
      }
    static const struct {
      const char* op;
      const char* c;
    } cmp[] = {{"CmpEq", "=="}, {"CmpNe", "!="}, {"CmpLt", "<"}, {"CmpLe", "<="}, {"CmpGt", ">"}, {"CmpGe", ">="}};
    for (const auto& u : cmp)
      if (op == u.op) {
        // eval_cmp (kernel_eval.rs:871-882): both operands at their own (common) type, 1 or 0.
        if (int_node_type(p.a[1], compute) != int_node_type(p.a[2], compute)) {
          why = "a comparison of operands of different types";
          return false;
        }
        if (!own(p.a[1], a) || !own(p.a[2], b)) return false;
        out = "(" + std::string(T) + ")((" + a + ") " + u.c + " (" + b + ") ? 1 : 0)";
        return true;
      }
    why = "the integer binary op " + op;
    return false;
  }
  if (tag == "Select") {
    // eval_int_select (kernel_eval.rs:850-860): the condition at its own type tested != 0, then
    // one arm evaluated at `t`.
    if (p.t != J::Arr || p.a.size() != 3 || !own(p.a[0], c) || !at(p.a[1], t, a) || !at(p.a[2], t, b)) return false;
    out = "((" + c + ") != 0 ? (" + a + ") : (" + b + "))";
    return true;
  }
  why = "the integer expression node " + tag;
  return false;
}

// True when evaluating `e` costs a library call or a division in f64: the per-element value
// is then worth holding in registers between a stage and the epilogue.
bool costly(const kir::J& e) {
  using kir::J;
  if (e.t != J::Obj || e.o.size() != 1) return false;
  const std::string& tag = e.o[0].first;
  const J& p = e.o[0].second;
  if (tag == "Unary" && p.t == J::Arr && !p.a.empty() && p.a[0].t == J::Str) {
    static const char* const cheap[] = {"Neg", "Abs", "Sqr", "Relu", "Floor", "Ceil", "Round", "Trunc", "Sign", "Step"};
    bool is_cheap = false;
    for (const char* c : cheap) is_cheap = is_cheap || p.a[0].s == c;
    if (!is_cheap) return true;
  }
  if (tag == "Binary" && p.t == J::Arr && !p.a.empty() && p.a[0].t == J::Str) {
    static const char* const dear[] = {"Pow", "Atan2", "Rem", "RemTrunc"};
    for (const char* c : dear)
      if (p.a[0].s == c) return true;
  }
  if (tag == "Div") return true;
  if (p.t == J::Arr)
    for (const J& x : p.a)
      if (costly(x)) return true;
  return false;
}

// True when the expression node `tag` occurs anywhere in `e`.
bool mentions(const kir::J& e, const char* tag) {
  using kir::J;
  if (e.t == J::Obj)
    for (const auto& kv : e.o)
      if (kv.first == tag || mentions(kv.second, tag)) return true;
  if (e.t == J::Arr)
    for (const J& x : e.a)
      if (mentions(x, tag)) return true;
  return false;
}

// True when `sub` occurs in `e` as a subtree.
bool contains(const kir::J& e, const kir::J& sub) {
  using kir::J;
  if (e == sub) return true;
  if (e.t == J::Obj)
    for (const auto& kv : e.o)
      if (contains(kv.second, sub)) return true;
  if (e.t == J::Arr)
    for (const J& x : e.a)
      if (contains(x, sub)) return true;
  return false;
}

}  // namespace

// A gather beyond OpDef::gather (kernel_lift/gather.rs:35-101): n inputs, the index and the
// gathered data among them, an elementwise body.  One lane per output element: the index at the
// output coordinate, its clamp and the policy as the cell does (:184-232), every other input read
// at the output coordinate (the gathered one at the clamped coordinate on the axis), the body
// evaluated in f64 and rounded once at the store, as the oracle evaluates a statement; a body that
// is a single input moves its bits.  Every buffer is addressed through its strides (dense ones
// with their row-major strides), so one entry serves pointer and storage-image launches.
int32_t lower_gather_x(const unp_form& f, const GatherExpr& gx, Lowered& L, std::string& why) {
  L = Lowered{};
  L.form = f;
  L.gx = gx;
  const int32_t n = gx.n_inputs, ix = gx.index_slot, data = f.data_slot;
  if (f.rank < 1 || f.rank > 8 || n < 2 || n > 8 || ix < 0 || ix >= n || data < 0 || data >= n || ix == data) {
    why = "an ill-formed gather";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (!oob_name(f.oob) || (f.index_dtype != UNP_I32 && f.index_dtype != UNP_I64 && f.index_dtype != UNP_U32)) {
    why = "an unknown out-of-range policy or a non-integer index";
    return UNP_UNSUPPORTED_KERNEL;
  }
  const kir::J& b = gx.body;
  const bool leaf = b.t == kir::J::Obj && b.o.size() == 1 && b.o[0].first == "Input" && b.o[0].second.is_int;
  const size_t eb = kind_bytes(f.dtype);
  const char* T = ctype(f.dtype);
  std::string value;
  if (leaf) {
    const int64_t k = b.o[0].second.i;
    if (k == ix) {
      why = "a gather whose body is its index";
      return UNP_UNSUPPORTED_KERNEL;
    }
    if (eb == 0) {
      why = "a gather of a sub-byte element kind";
      return UNP_UNSUPPORTED_DTYPE;
    }
    value = "v" + std::to_string(k);  // the raw element, moved as bits
  } else {
    if (f.dtype != UNP_F32 && f.dtype != UNP_F64) {
      why = "a gather body at " + std::string(kind_name(f.dtype)) + " (bodies are spelled at F32 and F64)";
      return UNP_UNSUPPORTED_DTYPE;
    }
    std::string e;
    if (!expr_cpp(b, T, e, why)) {
      why = "body: " + why + " has no spelling here";
      return UNP_UNSUPPORTED_OP;
    }
    value = "(" + std::string(T) + ")(" + e + ")";
  }
  const char* E = eb == 1 ? "unsigned char" : eb == 2 ? "unsigned short" : eb == 4 ? "unsigned int" : "unsigned long long";
  const char* I = ctype(f.index_dtype);
  std::ostringstream name;
  name << "unp_gather_x" << n << "_" << lower_name(f.dtype) << "_by_" << lower_name(f.index_dtype) << "_"
       << oob_name(f.oob) << "_" << std::hex << (fnv1a64(kir::write(b) + std::to_string(ix) + std::to_string(data)) & 0xffffffffu);
  L.name = name.str();
  L.threads = 256;
  L.blocks_per_cu = 8;
  L.scan_axis = 0;
  for (int32_t d = 0; d < f.rank; ++d)
    if ((f.axes_mask >> d) & 1u) L.scan_axis = d;
  std::ostringstream src;
  src << header(L.name, f);
  Entry e;
  e.fast = false;
  e.strided = false;
  e.vec = (int)eb;
  e.symbol = L.name + "_e";
  src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(";
  for (int k = 0; k < n; ++k) src << "const void* in" << k << ", ";
  src << "void* out, unp::gather_x_view v, " << I << " src_extent) {\n"
      << "  const long long stride = (long long)gridDim.x * blockDim.x;\n"
      << "  for (long long o = (long long)blockIdx.x * blockDim.x + threadIdx.x; o < v.outs; o += stride) {\n"
      << "    long long c[8], q = o, oo = 0;\n"
      << "    for (long long d = v.rank - 1; d >= 0; --d) { c[d] = q % v.ext[d]; q /= v.ext[d]; oo += c[d] * v.ostr[d]; }\n"
      << "    auto at = [&](int k) { long long s = 0; for (long long d = 0; d < v.rank; ++d) s += c[d] * v.istr[k][d]; return s; };\n"
      << "    const " << I << " raw = static_cast<const " << I << "*>(in" << ix << ")[at(" << ix << ")];\n"
      << "    const bool below = unp::below_zero(raw);\n"
      << "    const bool oob = below || !(raw < src_extent);\n";
  if (f.oob != UNP_OOB_CLAMP) {
    src << "    if (oob) {\n";
    if (f.oob == UNP_OOB_ZEROFILL) src << "      static_cast<" << E << "*>(out)[oo] = 0;\n";
    src << "      continue;\n    }\n";
  }
  src << "    const " << I << " cl = below ? (" << I << ")0 : (oob ? (" << I << ")(src_extent - (" << I << ")1) : raw);\n";
  for (int k = 0; k < n; ++k) {
    if (k == ix) continue;
    src << "    const long long off" << k << " = at(" << k << ")"
        << (k == data ? " + ((long long)cl - c[v.axis]) * v.istr[" + std::to_string(k) + "][v.axis]" : std::string())
        << ";\n";
    if (leaf) src << "    const " << E << " v" << k << " = static_cast<const " << E << "*>(in" << k << ")[off" << k << "];\n";
  }
  if (leaf) {
    src << "    static_cast<" << E << "*>(out)[oo] = " << value << ";\n";
  } else {
    src << "    double x[" << n << "];\n";
    for (int k = 0; k < n; ++k) {
      if (k == ix) src << "    x[" << k << "] = (double)raw;\n";
      else src << "    x[" << k << "] = (double)static_cast<const " << T << "*>(in" << k << ")[off" << k << "];\n";
    }
    src << "    static_cast<" << T << "*>(out)[oo] = " << value << ";\n";
  }
  src << "  }\n}\n";
  L.entries.push_back(e);
  Entry x = e;
  x.strided = true;  // the same entry reads storage images
  L.entries.push_back(x);
  L.source = src.str();
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"gather\",\"dtype\":\"" << kind_name(f.dtype)
    << "\",\"index_dtype\":\"" << kind_name(f.index_dtype) << "\",\"oob\":\"" << oob_name(f.oob)
    << "\",\"axis\":" << L.scan_axis << ",\"rank\":" << f.rank << ",\"inputs\":" << n << ",\"index_slot\":" << ix
    << ",\"data_slot\":" << data << ",\"body\":" << json_str(kir::write(b)) << ",\"params\":[";
  for (int k = 0; k < n; ++k)
    j << "{\"name\":\"in" << k << "\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\""
      << kind_name(k == ix ? f.index_dtype : f.dtype) << "\"},";
  j << "{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\"}";
  for (int d = 0; d < f.rank; ++d) j << ",{\"name\":\"n" << d << "\",\"kind\":\"scalar\",\"dtype\":\"I32\"}";
  j << ",{\"name\":\"src_extent\",\"kind\":\"scalar\",\"dtype\":\"" << kind_name(f.index_dtype)
    << "\"}],\"launch\":{\"block\":[256,1,1],\"grid\":\"cu_count*8\",\"grid_policy\":\"one lane per output "
       "element, lanes stride over the outputs\"},\"entries\":[{\"symbol\":\""
    << e.symbol << "\",\"when\":\"always (dense buffers with their row-major strides, storage images with theirs)\"}]"
    << ",\"workspace\":null,\"compiler_args\":[\"--offload-arch=gfx950\",\"-O3\",\"-Xclang\",\"-target-feature\",\"-Xclang\",\"-packed-fp32-ops\"]"
    << ",\"fidelity_notes\":["
    << json_str(leaf ? "a raw bit move: bit-exact for every grid and block"
                     : "the body evaluated in f64 and rounded once at the store, as the oracle evaluates a statement; "
                       "bit-exact against the oracle")
    << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

// An Access::Elementwise lift (kernel_lift.rs:96-153): out[c] = body(in0[c], ..., in(n-1)[c]) at
// every output coordinate c, input k read through its axis permutation when it has one.  The cell
// follows the oracle's statement model (launch_cases.rs:14-27): a float body is evaluated in f64 and
// rounded once at the store (bit-exact against the oracle, so 0 ULPs on every corpus case, the
// IEEE-rounded divide included); an integer body at I32/I64/U32/U64 by the total rule (unp::xi);
// a body that is one input moves that input's bits at any element kind of whole bytes.
// Entries: `_v` streams 16-byte packs when every buffer is dense, unpermuted and 16-byte aligned,
// `_s` the same element by element at any alignment, and `_e` walks each buffer through its own
// strides (a permuted input, or storage images that are not dense row-major).
int32_t lower_elementwise(const unp_form& f, const ElementwiseExpr& ew, Lowered& L, std::string& why) {
  L = Lowered{};
  L.form = f;
  L.form.kind = UNP_FORM_ELEMENTWISE;
  L.ew = ew;
  const int32_t n = ew.n_inputs;
  if (f.rank < 1 || f.rank > 8 || n < 1 || n > 8) {
    why = "an elementwise op of 1 to 8 inputs at rank 1 to 8";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (!ew.perms.empty() && ew.perms.size() != (size_t)n) {
    why = "an ill-formed view";
    return UNP_UNSUPPORTED_KERNEL;
  }
  const kir::J& b = ew.body;
  const bool leaf = b.t == kir::J::Obj && b.o.size() == 1 && b.o[0].first == "Input" && b.o[0].second.is_int;
  const size_t eb = kind_bytes(f.dtype);
  std::string T, cell;
  const bool is_float = f.dtype == UNP_F32 || f.dtype == UNP_F64;
  if (leaf) {
    if (eb == 0) {
      why = "an elementwise op over a sub-byte element kind";
      return UNP_UNSUPPORTED_DTYPE;
    }
    T = eb == 1 ? "unsigned char" : eb == 2 ? "unsigned short" : eb == 4 ? "unsigned int" : eb == 8 ? "unsigned long long" : "uint4";
    cell = "  return a[" + std::to_string(b.o[0].second.i) + "];\n";
  } else if (is_float) {
    T = ctype(f.dtype);
    std::string e;
    if (!expr_cpp(b, T.c_str(), e, why)) {
      why = "body: " + why + " has no spelling here";
      return UNP_UNSUPPORTED_OP;
    }
    cell = "  double x[" + std::to_string(n) + "];\n  for (int k = 0; k < " + std::to_string(n) +
           "; ++k) x[k] = (double)a[k];\n  return (" + T + ")(" + e + ");\n";
  } else if (int_ctype(f.dtype)) {
    T = int_ctype(f.dtype);
    std::string e;
    if (int_node_type(b, f.dtype) != f.dtype) {
      why = "body: an integer expression whose type is not the compute dtype (or a node outside the integer "
            "evaluator's subset: ConstInt, Cast, Add, Sub, Mul, Div, Shl, Shr, Min, Max, BitAnd, BitOr, BitXor, "
            "comparisons and Select)";
      return UNP_UNSUPPORTED_OP;
    }
    if (!int_expr_cpp(b, f.dtype, f.dtype, e, why)) {
      why = "body: " + why + " has no spelling here";
      return UNP_UNSUPPORTED_OP;
    }
    cell = "  const " + T + "* x = a;\n  return " + e + ";\n";
  } else {
    why = std::string("an elementwise body at ") + (kind_name(f.dtype) ? kind_name(f.dtype) : "an unknown kind") +
          " (bodies are spelled at F32, F64, I32, I64, U32 and U64; a single-input body at any whole-byte kind)";
    return UNP_UNSUPPORTED_DTYPE;
  }
  std::string perm_text;
  for (const auto& p : ew.perms) {
    perm_text += "[";
    for (size_t d = 0; d < p.size(); ++d) perm_text += (d ? "," : "") + std::to_string(p[d]);
    perm_text += "]";
  }
  const int vec = eb && eb <= 16 ? (int)(16 / eb) : 1;
  std::ostringstream name;
  name << "unp_ew" << n << "_" << lower_name(f.dtype) << "_" << std::hex
       << (fnv1a64(kir::write(b) + "|" + perm_text + "|" + std::to_string(f.rank)) & 0xffffffffu);
  L.name = name.str();
  L.threads = 256;
  L.blocks_per_cu = 8;
  const std::string N = std::to_string(n);
  auto loads = [&](const std::string& idx_of_k) {
    std::string s = "{";
    for (int k = 0; k < n; ++k) {
      std::string ix = idx_of_k;
      for (size_t at = ix.find('#'); at != std::string::npos; at = ix.find('#')) ix.replace(at, 1, std::to_string(k));
      s += (k ? ", " : "") + ix;
    }
    return s + "}";
  };
  auto params = [&]() {
    std::string s;
    for (int k = 0; k < n; ++k) s += "const void* in" + std::to_string(k) + ", ";
    return s + "void* out";
  };
  std::ostringstream src;
  src << header(L.name, L.form) << "namespace {\n"
      << "using ew_t = " << T << ";\n"
      << "__device__ __forceinline__ ew_t ew_cell(const ew_t (&a)[" << N << "]) {\n"
      << cell << "}\n"
      << "struct alignas(16) ew_pack { ew_t e[" << vec << "]; };\n"
      << "}  // namespace\n";
  const std::string V = L.name + "_v", S = L.name + "_s", E = L.name + "_e";
  src << "extern \"C\" __global__ void " << kLaunchBounds << " " << V << "(" << params() << ", long long n) {\n"
      << "  const long long stride = (long long)gridDim.x * blockDim.x;\n"
      << "  const long long t0 = (long long)blockIdx.x * blockDim.x + threadIdx.x;\n"
      << "  const long long np = n / " << vec << ";\n"
      << "  for (long long i = t0; i < np; i += stride) {\n";
  for (int k = 0; k < n; ++k)
    src << "    const ew_pack p" << k << " = static_cast<const ew_pack*>(in" << k << ")[i];\n";
  src << "    ew_pack o;\n"
      << "#pragma unroll\n"
      << "    for (int j = 0; j < " << vec << "; ++j) {\n"
      << "      const ew_t a[" << N << "] = " << loads("p#.e[j]") << ";\n"
      << "      o.e[j] = ew_cell(a);\n"
      << "    }\n"
      << "    static_cast<ew_pack*>(out)[i] = o;\n"
      << "  }\n"
      << "  for (long long i = np * " << vec << " + t0; i < n; i += stride) {\n"
      << "    const ew_t a[" << N << "] = " << loads("static_cast<const ew_t*>(in#)[i]") << ";\n"
      << "    static_cast<ew_t*>(out)[i] = ew_cell(a);\n"
      << "  }\n}\n";
  src << "extern \"C\" __global__ void " << kLaunchBounds << " " << S << "(" << params() << ", long long n) {\n"
      << "  const long long stride = (long long)gridDim.x * blockDim.x;\n"
      << "  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {\n"
      << "    const ew_t a[" << N << "] = " << loads("static_cast<const ew_t*>(in#)[i]") << ";\n"
      << "    static_cast<ew_t*>(out)[i] = ew_cell(a);\n"
      << "  }\n}\n";
  // The strided entry: v.ext the output's extents, v.ostr its strides, v.istr[k] input k's strides
  // over the output's axes (a permuted input's strides already permuted by the host).
  src << "extern \"C\" __global__ void " << kLaunchBounds << " " << E << "(" << params()
      << ", unp::gather_x_view v) {\n"
      << "  const long long stride = (long long)gridDim.x * blockDim.x;\n"
      << "  for (long long o = (long long)blockIdx.x * blockDim.x + threadIdx.x; o < v.outs; o += stride) {\n"
      << "    long long q = o, oo = 0, off[" << N << "] = {};\n"
      << "    for (long long d = v.rank - 1; d >= 0; --d) {\n"
      << "      const long long c = q % v.ext[d];\n"
      << "      q /= v.ext[d];\n"
      << "      oo += c * v.ostr[d];\n"
      << "#pragma unroll\n"
      << "      for (int k = 0; k < " << N << "; ++k) off[k] += c * v.istr[k][d];\n"
      << "    }\n"
      << "    const ew_t a[" << N << "] = " << loads("static_cast<const ew_t*>(in#)[off[#]]") << ";\n"
      << "    static_cast<ew_t*>(out)[oo] = ew_cell(a);\n"
      << "  }\n}\n";
  Entry ev;
  ev.symbol = V;
  ev.fast = true;
  ev.vec = vec;
  Entry es = ev;
  es.symbol = S;
  es.fast = false;
  es.vec = 1;
  Entry ee = es;
  ee.symbol = E;
  ee.strided = true;
  L.entries = {ev, es, ee};
  L.source = src.str();
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"elementwise\",\"dtype\":\"" << kind_name(f.dtype)
    << "\",\"rank\":" << f.rank << ",\"inputs\":" << n << ",\"body\":" << json_str(kir::write(b)) << ",\"views\":[";
  for (size_t k = 0; k < ew.perms.size(); ++k) {
    j << (k ? "," : "") << "{\"Permute\":{\"perm\":[";
    for (size_t d = 0; d < ew.perms[k].size(); ++d) j << (d ? "," : "") << ew.perms[k][d];
    j << "]}}";
  }
  j << "],\"params\":[";
  for (int k = 0; k < n; ++k)
    j << "{\"name\":\"in" << k << "\",\"kind\":\"buffer\",\"role\":\"Read\",\"dtype\":\"" << kind_name(f.dtype) << "\"},";
  j << "{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\",\"dtype\":\"" << kind_name(f.dtype) << "\"}";
  for (int d = 0; d < f.rank; ++d) j << ",{\"name\":\"n" << d << "\",\"kind\":\"scalar\",\"dtype\":\"I32\"}";
  j << "],\"launch\":{\"block\":[256,1,1],\"grid\":\"min(cu_count*8, the lanes the elements need)\",\"grid_policy\":"
       "\"lanes stride over the elements (16-byte packs on the _v entry)\"},\"entries\":["
    << "{\"symbol\":\"" << V << "\",\"when\":\"every buffer dense row-major, no permuted input, every base 16-byte aligned\"},"
    << "{\"symbol\":\"" << S << "\",\"when\":\"every buffer dense row-major and no permuted input, any alignment\"},"
    << "{\"symbol\":\"" << E << "\",\"when\":\"a permuted input, or storage images that are not dense row-major\"}]"
    << ",\"workspace\":null,\"compiler_args\":[\"--offload-arch=gfx950\",\"-O3\",\"-Xclang\",\"-target-feature\",\"-Xclang\",\"-packed-fp32-ops\"]"
    << ",\"fidelity_notes\":["
    << json_str(leaf ? "a raw bit move: bit-exact for every grid and block"
                : is_float ? "the body evaluated in f64 and rounded once at the store, as the oracle evaluates a "
                             "statement: bit-exact against the oracle (0 ULPs, the divide IEEE-rounded)"
                           : "integer arithmetic by the total rule (Add/Sub/Mul wrap; a zero divisor and signed MIN / -1 "
                             "give the dividend; shift counts modulo the width): bit-exact against the oracle")
    << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

int32_t lower_row_reduce(const RowReduceSpec& sp, Lowered& L, std::string& why) {
  L = Lowered{};
  L.form.kind = UNP_FORM_ROW_REDUCE;
  L.form.dtype = sp.dtype;
  L.form.rank = sp.rank;
  L.rr = sp;
  if (sp.dtype != UNP_F32 && sp.dtype != UNP_F64) {
    why = "a row reduction outside F32 and F64";
    return UNP_UNSUPPORTED_DTYPE;
  }
  const size_t NS = sp.ops.size();
  if (NS == 0 || NS != sp.pres.size() || sp.n_inputs < 1 || sp.n_inputs > 8) {
    why = "a row reduction needs 1 to 8 inputs and at least one stage";
    return UNP_UNSUPPORTED_KERNEL;
  }
  for (int32_t op : sp.ops)
    if (op == UNP_OP_PROD) {
      why = "a Prod stage (a float product is not order-independent and declares no bound)";
      return UNP_UNSUPPORTED_KERNEL;
    }
  const char* T = ctype(sp.dtype);
  std::vector<std::string> pre(NS);
  std::string epi;
  for (size_t st = 0; st < NS; ++st)
    if (!expr_cpp(sp.pres[st], T, pre[st], why)) {
      why = "stage " + std::to_string(st) + ": " + why + " has no spelling here";
      return UNP_UNSUPPORTED_OP;
    }
  if (!expr_cpp(sp.epilogue, T, epi, why)) {
    why = "epilogue: " + why + " has no spelling here";
    return UNP_UNSUPPORTED_OP;
  }
  // A stage whose pre expression is costly and recurs in the epilogue (softmax's exp(x - max)):
  // the register-resident entries keep its per-element f64 value from the stage and the
  // epilogue reads it back.  It is the same f64 expression of the same operands, so the result
  // is unchanged; only the second evaluation is saved.
  int cached = -1;
  std::string epi_c = epi;
  for (size_t st = 0; st < NS && cached < 0; ++st)
    if (costly(sp.pres[st]) && contains(sp.epilogue, sp.pres[st])) {
      std::string w2;
      if (!expr_cpp(sp.epilogue, T, epi_c, w2, &sp.pres[st])) {
        why = "epilogue: " + w2 + " has no spelling here";
        return UNP_UNSUPPORTED_OP;
      }
      cached = (int)st;
    }
  // An f32 epilogue that is a quotient by a row value and reuses a costly stage value (softmax's
  // exp(x - max) / sum, whose per-element f64 work bounds the kernel rather than HBM): the
  // element multiplies by the row's reciprocal, which the compiler computes once per row, in
  // place of an IEEE f64 division per element.  A memory-bound quotient (RMS norm, a centred
  // quotient) keeps its division: the rewrite would buy it no time.  x * (1 / s) is within 2^-52 of x / s, so after the
  // one rounding to f32 the output is the quotient's or its neighbour (1 ulp, only where the
  // quotient lies that close to a rounding boundary), inside the 2-ulp tolerance of an f32
  // epilogue (kernel_row_reduce_agrees.rs:25).  Zero, infinite and NaN divisors give the same
  // results either way.  Only a division at the root, whose value goes straight to the store,
  // is rewritten: under a comparison or another op, a 1-ulp change could move more than 1 ulp.
  bool recip = false;
  if (sp.dtype == UNP_F32 && cached >= 0 && sp.epilogue.t == kir::J::Obj && sp.epilogue.o.size() == 1 &&
      sp.epilogue.o[0].first == "Div" && sp.epilogue.o[0].second.t == kir::J::Arr &&
      sp.epilogue.o[0].second.a.size() == 2 && !mentions(sp.epilogue.o[0].second.a[1], "Input")) {
    const kir::J& num = sp.epilogue.o[0].second.a[0];
    const kir::J& den = sp.epilogue.o[0].second.a[1];
    std::string a, b, ac, w2;
    const kir::J* reuse = cached >= 0 ? &sp.pres[cached] : nullptr;
    if (expr_cpp(num, T, a, w2) && expr_cpp(den, T, b, w2) && expr_cpp(num, T, ac, w2, reuse)) {
      epi = "(" + a + " * (1.0 / " + b + "))";
      epi_c = "(" + ac + " * (1.0 / " + b + "))";
      recip = true;
    }
  }
  // The name carries a hash of the expressions: different row reductions never share a symbol.
  std::string key = std::string(T) + "|" + std::to_string(sp.n_inputs);
  for (size_t st = 0; st < NS; ++st) key += "|" + std::to_string(sp.ops[st]) + ":" + pre[st];
  key += "|" + epi;
  char hx[17];
  std::snprintf(hx, sizeof hx, "%016llx", (unsigned long long)fnv1a64(key));
  L.name = std::string("unp_row_reduce_") + lower_name(sp.dtype) + "_s" + std::to_string(NS) + "_" + std::string(hx, 8);
  const std::string ops = L.name + "_ops";
  std::ostringstream src;
  unp_form f{};
  f.kind = UNP_FORM_ROW_REDUCE;
  src << header(L.name, f);
  src << "struct " << ops << " {\n  static constexpr int op[" << NS << "] = {";
  for (size_t st = 0; st < NS; ++st) src << (st ? ", " : "") << sp.ops[st];
  src << "};\n  static constexpr int cached = " << cached << ";\n"
      << "  template <int S> static __device__ __forceinline__ double pre(const double* x, const double* r);\n"
      << "  static __device__ __forceinline__ double epi(const double* x, const double* r) { (void)x; (void)r; return "
      << epi << "; }\n"
      << "  static __device__ __forceinline__ double epi_c(const double* x, const double* r, double c) { (void)x; (void)r; "
      << "(void)c; return " << epi_c << "; }\n};\n";
  for (size_t st = 0; st < NS; ++st)
    src << "template <> __device__ __forceinline__ double " << ops << "::pre<" << st
        << ">(const double* x, const double* r) { (void)x; (void)r; return " << pre[st] << "; }\n";
  const int vec = vec_of(sp.dtype);
  struct E {
    const char* suffix;
    int vec, r;
    bool fast;
  } es[] = {{"_c4", vec, 4, true}, {"_c", vec, 8, true}, {"_v", vec, 0, true}, {"_s", 1, 0, false}};
  for (const E& e : es) {
    Entry en;
    en.symbol = L.name + e.suffix;
    en.vec = e.vec;
    en.k = e.r;  // vectors per thread held in registers (0: re-read)
    en.fast = e.fast;
    src << "extern \"C\" __global__ void " << kLaunchBounds << " " << en.symbol << "(";
    for (int k = 0; k < sp.n_inputs; ++k) src << "const " << T << "* in" << k << ", ";
    src << T << "* out, long long rows, long long cols) {\n  const " << T << "* in[" << sp.n_inputs << "] = {";
    for (int k = 0; k < sp.n_inputs; ++k) src << (k ? ", " : "") << "in" << k;
    src << "};\n  unp::row_reduce_staged<" << T << ", " << sp.n_inputs << ", " << NS << ", " << ops << ", 256, " << e.vec
        << ", " << e.r << ">(in, out, rows, cols);\n}\n";
    L.entries.push_back(en);
  }
  L.source = src.str();
  L.threads = 256;
  L.blocks_per_cu = 8;
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"row_reduce\",\"dtype\":\"" << kind_name(sp.dtype)
    << "\",\"rank\":" << sp.rank << ",\"inputs\":" << sp.n_inputs << ",\"stages\":[";
  static const char* const opn[] = {"Sum", "Prod", "Max", "Min", "Mean"};
  for (size_t st = 0; st < NS; ++st)
    j << (st ? "," : "") << "{\"op\":\"" << opn[sp.ops[st]] << "\",\"pre\":" << json_str(pre[st]) << "}";
  j << "],\"epilogue\":" << json_str(epi) << ",\"epilogue_reuses_stage\":" << cached << ",\"params\":[";
  for (int k = 0; k < sp.n_inputs; ++k) j << "{\"name\":\"in" << k << "\",\"kind\":\"buffer\",\"role\":\"Read\"},";
  j << "{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\"}";
  for (int d = 0; d < sp.rank; ++d) j << ",{\"name\":\"n" << d << "\",\"kind\":\"scalar\",\"dtype\":\"I32\"}";
  j << "],\"launch\":{\"block\":[256,1,1],\"grid\":\"cu_count*min(8, blocks one CU holds)\",\"grid_policy\":\"one "
       "block per row, rows block-strided; the next row's loads issued before this row's stages\"},\"entries\":[";
  for (size_t i = 0; i < L.entries.size(); ++i)
    j << (i ? "," : "") << "{\"symbol\":\"" << L.entries[i].symbol << "\",\"vec\":" << L.entries[i].vec
      << ",\"row_in_registers\":" << (L.entries[i].k ? "true" : "false") << ",\"when\":\""
      << (L.entries[i].k == 4 ? "cols % vec == 0, every buffer 16-byte aligned and cols <= 256 * vec * 4"
          : L.entries[i].k     ? "cols % vec == 0, every buffer 16-byte aligned and 256 * vec * 4 < cols <= 256 * vec * 8"
                               : (L.entries[i].fast ? "cols % vec == 0 and every buffer 16-byte aligned" : "otherwise"))
      << "\"}";
  j << "],\"workspace\":null"
    << ",\"compiler_args\":[\"--offload-arch=gfx950\",\"-O3\",\"-Xclang\",\"-target-feature\",\"-Xclang\",\"-packed-fp32-ops\"]"
    << ",\"fidelity_notes\":["
    << json_str("expressions evaluate in f64 and round once per statement, as the kernel evaluator runs the lifted "
                "kernel; +, -, *, /, fma, sqrt and the comparisons are exact, the device's f64 transcendentals are "
                "within an ulp of the host libm's")
    << "," << json_str("Sum/Mean stages fold in f64 in a geometry-fixed order: within the declared bound "
                       "gamma_(n-1)*sum|x| of the serial fold, then one rounding; Max/Min stages are exact except NaN "
                       "payload and the sign of a zero");
  if (recip)
    j << "," << json_str("the f32 epilogue's quotient by a row value multiplies by the row's f64 reciprocal: "
                         "within 2^-52 of the quotient, so the f32 output is the quotient's rounding or its "
                         "neighbour, within the 2-ulp tolerance of an f32 epilogue");
  j << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

namespace {

// The pre-map and post of a reduction or scan as C++ expressions over x[k] (the inputs) and r[0]
// (the rounded fold): in f64 for F32/F64, at the element type by the total integer rule for
// I32/I64 (no post there).  False, with `why` set, for a node that has no spelling.
bool pre_ops_cpp(int32_t dtype, const ReductionExpr& rx, std::string& pre, std::string& post, std::string& why) {
  if (dtype == UNP_I32 || dtype == UNP_I64) {
    if (int_node_type(rx.body, dtype) != dtype || !int_expr_cpp(rx.body, dtype, dtype, pre, why)) {
      if (why.empty()) why = "an integer expression whose type is not the compute dtype";
      why = "body: " + why + " has no spelling here";
      return false;
    }
    return true;
  }
  if (!expr_cpp(rx.body, ctype(dtype), pre, why)) {
    why = "body: " + why + " has no spelling here";
    return false;
  }
  if (rx.has_post && !expr_cpp(rx.post, ctype(dtype), post, why)) {
    why = "post: " + why + " has no spelling here";
    return false;
  }
  return true;
}

// The OPS struct the xreduce / xscan templates take: `arg` the type the expressions read their
// inputs at and `acc` the fold's (double for a float, the element type for an integer).  A scan's
// post also reads the position's inputs.
std::string pre_ops_struct(const std::string& ops, int32_t dtype, bool has_post, const std::string& pre,
                           const std::string& post, bool scan) {
  const bool is_int = dtype == UNP_I32 || dtype == UNP_I64;
  const std::string A = is_int ? ctype(dtype) : "double";
  std::ostringstream s;
  s << "struct " << ops << " {\n  typedef " << A << " arg;\n  typedef " << A << " acc;\n"
    << "  static constexpr bool has_post = " << (has_post ? "true" : "false") << ";\n"
    << "  static __device__ __forceinline__ " << A << " pre(const " << A << "* x) { (void)x; return " << pre << "; }\n"
    << "  static __device__ __forceinline__ " << A << " post(const " << A << "* r" << (scan ? ", const " + A + "* x" : "")
    << ") { (void)r; " << (scan ? "(void)x; " : "") << "return " << post << "; }\n};\n";
  return s.str();
}

}  // namespace

int32_t lower_reduction_x(const unp_form& f, const ReductionExpr& rx, Lowered& L, std::string& why) {
  if (rx.plain) return lower_form(f, L, why);
  L = Lowered{};
  L.form = f;
  L.rx = rx;
  if (f.rank < 1 || f.rank > 8) {
    why = "rank is zero or more than 8";
    return UNP_LIFT_DECLINE;
  }
  // The integer kinds the reference lifts a body at (kernel_lift.rs:755-800): I32 and I64, with the
  // identity post.
  const bool int_body = f.dtype == UNP_I32 || f.dtype == UNP_I64;
  if (f.dtype != UNP_F32 && f.dtype != UNP_F64 && !int_body) {
    why = "a reduction with a pre-map body or a fused post outside F32, F64, I32 and I64";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (int_body && rx.has_post) {
    why = "a fused post at an integer dtype";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (rx.n_inputs < 1 || rx.n_inputs > 8) {
    why = "a reduction reads 1 to 8 inputs";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (!reduction_ok(f.dtype, f.op0, why)) return UNP_UNSUPPORTED_KERNEL;
  if (f.op0 == UNP_OP_PROD && !int_body) {
    why = "a float Prod with a pre-map body or a fused post (not order-independent, and no declared bound)";
    return UNP_UNSUPPORTED_KERNEL;
  }
  const uint32_t mask = reduction_mask(f);
  if (mask == 0 || (mask >> f.rank) != 0) {
    why = "a reduced axis outside the rank";
    return UNP_LIFT_DECLINE;
  }
  const char sched = reduction_schedule(mask, f.rank);
  L.axes_mask = mask;
  L.red_schedule = sched;
  L.reduce_all = sched == 'a';
  L.form.reduced_from = f.rank;
  for (int32_t d = f.rank - 1; d >= 0 && ((mask >> d) & 1u); --d) L.form.reduced_from = d;
  const char* T = ctype(f.dtype);
  std::string pre, post = "r[0]";
  if (!pre_ops_cpp(f.dtype, rx, pre, post, why)) return UNP_UNSUPPORTED_OP;
  const int NI = rx.n_inputs;
  const std::string key = std::string(T) + "|" + std::to_string(NI) + "|" + std::to_string(f.op0) + "|" + sched +
                          "|" + pre + "|" + (rx.has_post ? post : std::string("-"));
  char hx[17];
  std::snprintf(hx, sizeof hx, "%016llx", (unsigned long long)fnv1a64(key));
  L.name = std::string("unp_xreduce_") + op_name(f.op0) + "_" + lower_name(f.dtype) + "_" + std::string(hx, 8);
  const std::string ops = L.name + "_ops";
  std::ostringstream src;
  src << header(L.name, f) << pre_ops_struct(ops, f.dtype, rx.has_post, pre, post, false);
  auto sig = [&](std::ostringstream& o) {
    for (int k = 0; k < NI; ++k) o << "const " << T << "* in" << k << ", ";
    o << T << "* out";
  };
  auto ins = [&](std::ostringstream& o) {
    o << "  const " << T << "* in[" << NI << "] = {";
    for (int k = 0; k < NI; ++k) o << (k ? ", " : "") << "in" << k;
    o << "};\n";
  };
  const int V = vec_of(f.dtype);
  L.threads = 256;
  if (sched == 'r') {
    L.blocks_per_cu = 8;
    for (int fast = 1; fast >= 0; --fast) {
      Entry e;
      e.fast = fast;
      e.vec = fast ? V : 1;
      e.symbol = L.name + (fast ? "_xwv" : "_xws");
      src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(";
      sig(src);
      src << ", long long rows, long long cols) {\n";
      ins(src);
      src << "  unp::xreduce_rows<" << T << ", " << NI << ", " << f.op0 << ", " << ops << ", " << e.vec << ", 256, "
          << (fast ? 4 : 8) << ">(in, out, rows, cols);\n}\n";
      L.entries.push_back(e);
    }
  } else if (sched == 'a') {
    L.threads = 512;
    L.blocks_per_cu = 1;
    for (int fast = 1; fast >= 0; --fast) {
      Entry e;
      e.fast = fast;
      e.vec = fast ? V : 1;
      e.symbol = L.name + (fast ? "_xav" : "_xas");
      src << "extern \"C\" __global__ void __launch_bounds__(512) " << e.symbol << "(";
      sig(src);
      src << ", long long n, unsigned long long* partials, unsigned* counter, unsigned epoch, unp::waits wt) {\n";
      ins(src);
      src << "  unp::xreduce_all<" << T << ", " << NI << ", " << f.op0 << ", " << ops << ", " << e.vec << ", 512, "
          << (fast ? 8 : 8) << ">(in, out, n, partials, counter, epoch, wt);\n}\n";
      L.entries.push_back(e);
    }
  } else {
    L.blocks_per_cu = 8;
    Entry e;
    e.fast = false;
    e.vec = 1;
    e.symbol = L.name + "_xg";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(";
    sig(src);
    src << ", unp::axes_desc d) {\n";
    ins(src);
    src << "  unp::xreduce_generic<" << T << ", " << NI << ", " << f.op0 << ", " << ops << ", 256>(in, out, d);\n}\n";
    L.entries.push_back(e);
  }
  L.source = src.str();
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"reduction\",\"dtype\":\"" << kind_name(f.dtype)
    << "\",\"ops\":[\"" << op_name(f.op0) << "\"],\"rank\":" << f.rank << ",\"inputs\":" << NI << ",\"reduced_axes\":[";
  for (int32_t d = 0, n = 0; d < f.rank; ++d)
    if ((mask >> d) & 1u) j << (n++ ? "," : "") << d;
  j << "],\"schedule\":\"" << (sched == 'a' ? "all" : sched == 'r' ? "rows" : "generic") << "\",\"body\":" << json_str(pre)
    << ",\"post\":" << (rx.has_post ? json_str(post) : std::string("null")) << ",\"params\":[";
  for (int k = 0; k < NI; ++k) j << "{\"name\":\"in" << k << "\",\"kind\":\"buffer\",\"role\":\"Read\"},";
  j << "{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\"}";
  for (int d = 0; d < f.rank; ++d) j << ",{\"name\":\"n" << d << "\",\"kind\":\"scalar\",\"dtype\":\"I32\"}";
  j << "],\"launch\":{\"block\":[" << L.threads << ",1,1],\"grid_policy\":\""
    << (sched == 'r'   ? "one wave per row, waves stride over rows"
        : sched == 'a' ? "blocks stride over 16-byte vectors of every input, last-ticket block folds the partials"
                       : "one wave per output element, lanes stride over the reduced positions")
    << "\"},\"entries\":[";
  for (size_t i = 0; i < L.entries.size(); ++i)
    j << (i ? "," : "") << "{\"symbol\":\"" << L.entries[i].symbol << "\",\"vec\":" << L.entries[i].vec
      << ",\"when\":\""
      << (sched == 'm' || sched == 'g' ? "always"
          : L.entries[i].fast         ? "reduced extent % vec == 0 and every input 16-byte aligned"
                                      : "otherwise")
      << "\"}";
  j << "],\"workspace\":" << (sched == 'a' ? "{\"partials\":\"grid * 16 (f64, tagged with the launch epoch)\",\"counter\":4,\"stall\":4,\"host_state\":[\"epoch\"]}" : "null")
    << ",\"compiler_args\":[\"--offload-arch=gfx950\",\"-O3\",\"-Xclang\",\"-target-feature\",\"-Xclang\",\"-packed-fp32-ops\"]"
    << ",\"fidelity_notes\":["
    << json_str(int_body ? "the body evaluates at the element type by the total integer rule (Add/Sub/Mul wrap, a zero "
                           "divisor and MIN / -1 give the dividend, shift counts modulo the width) and the fold wraps at "
                           "the element type: every order gives the serial kernel's bits"
                         : "the body and the post evaluate in f64 and round once per statement, as the kernel evaluator "
                           "runs the lifted kernel; the fold is in f64 in a geometry-fixed order: a Sum/Mean within the "
                           "declared bound gamma_(n-1)*sum|x| of the serial fold, a Max/Min exact except NaN payload and "
                           "the sign of a zero")
    << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

// A scan with a pre-map body over n inputs and a fused post (lift_scan_opdef with pre and post,
// kernel_lift.rs:504-602; scan_launched.rs:54-102).  Float dtypes only: the expressions are
// spelled in f64.  The innermost axis with Sum / Max / Min runs the register look-back scan
// (xscan_lookback); any other axis, a Mean, a float Prod and the serial schedule run xscan_seq
// in the serial lift's order.
int32_t lower_scan_x(const unp_form& f, const ReductionExpr& rx, Lowered& L, std::string& why) {
  if (rx.plain) return lower_form(f, L, why);
  L = Lowered{};
  L.form = f;
  L.rx = rx;
  if (f.rank < 1 || f.rank > 8) {
    why = "rank is zero or more than 8";
    return UNP_LIFT_DECLINE;
  }
  // I32 and I64 take a pre-map with the identity post and no Mean (kernel_lift.rs:755-800).
  const bool int_body = f.dtype == UNP_I32 || f.dtype == UNP_I64;
  if (f.dtype != UNP_F32 && f.dtype != UNP_F64 && !int_body) {
    why = "a scan with a pre-map body or a fused post outside F32, F64, I32 and I64";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (int_body && (rx.has_post || f.op0 == UNP_OP_MEAN)) {
    why = rx.has_post ? "a fused post at an integer dtype" : "an integer Mean";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (rx.n_inputs < 1 || rx.n_inputs > 8) {
    why = "a scan reads 1 to 8 inputs";
    return UNP_UNSUPPORTED_KERNEL;
  }
  if (f.op0 != UNP_OP_SUM && f.op0 != UNP_OP_MAX && f.op0 != UNP_OP_MIN && f.op0 != UNP_OP_PROD &&
      f.op0 != UNP_OP_MEAN) {
    why = "a scan folds Sum, Prod, Max, Min or Mean";
    return UNP_UNSUPPORTED_KERNEL;
  }
  int32_t axis = f.rank - 1;
  if (f.axes_mask) {
    if ((f.axes_mask & (f.axes_mask - 1)) != 0 || (f.axes_mask >> f.rank) != 0) {
      why = "a scan scans exactly one axis inside the rank";
      return UNP_LIFT_DECLINE;
    }
    axis = __builtin_ctz(f.axes_mask);
  }
  // The fixed schedule folds the register look-back's carries in groups of 64 tiles in an order
  // the tiling fixes (lookback_grouped), as the plain scan's does.
  // An integer Prod wraps, so its look-back is exact in any order; a float Prod rounds at every
  // step and runs the serial order.
  const bool serial = axis != f.rank - 1 || (f.op0 == UNP_OP_PROD && !int_body) || f.op0 == UNP_OP_MEAN ||
                      f.schedule == UNP_SCHEDULE_SERIAL;
  const bool fixed = !serial && f.schedule == UNP_SCHEDULE_FIXED;
  L.serial_scan = serial;
  L.scan_axis = axis;
  const char* T = ctype(f.dtype);
  std::string pre, post = "r[0]";
  if (!pre_ops_cpp(f.dtype, rx, pre, post, why)) return UNP_UNSUPPORTED_OP;
  const int NI = rx.n_inputs;
  const char* EX = f.exclusive ? "true" : "false";
  const char* RV = f.reverse ? "true" : "false";
  const std::string key = std::string(T) + "|" + std::to_string(NI) + "|" + std::to_string(f.op0) + "|" + EX + "|" +
                          RV + "|" + (serial ? "q" : fixed ? "f" : "d") + "|" + pre + "|" +
                          (rx.has_post ? post : std::string("-"));
  char hx[17];
  std::snprintf(hx, sizeof hx, "%016llx", (unsigned long long)fnv1a64(key));
  L.name = std::string("unp_xscan_") + (serial ? "seq_" : fixed ? "fix_" : "") + (f.exclusive ? "excl_" : "incl_") +
           (f.reverse ? "rev_" : "") + op_name(f.op0) + "_" + lower_name(f.dtype) + "_" + std::string(hx, 8);
  const std::string ops = L.name + "_ops";
  std::ostringstream src;
  src << header(L.name, f) << pre_ops_struct(ops, f.dtype, rx.has_post, pre, post, true);
  std::ostringstream sig, ins;
  for (int k = 0; k < NI; ++k) sig << "const " << T << "* in" << k << ", ";
  sig << T << "* out";
  ins << "  const " << T << "* in[" << NI << "] = {";
  for (int k = 0; k < NI; ++k) ins << (k ? ", " : "") << "in" << k;
  ins << "};\n";
  Entry e;
  e.fast = false;
  e.vec = 1;
  if (serial) {
    e.threads = 256;
    e.blocks_per_cu = 8;
    e.symbol = L.name + "_xq";
    src << "extern \"C\" __global__ void __launch_bounds__(256) " << e.symbol << "(" << sig.str()
        << ", long long A, long long S, long long B) {\n" << ins.str() << "  unp::xscan_seq<" << T << ", " << NI
        << ", " << f.op0 << ", " << ops << ", " << EX << ", " << RV << ">(in, out, A, S, B);\n}\n";
  } else {
    // 8 waves of K = 8 steps: a 4096-position block tile, the raw inputs of every step kept in
    // registers for the post.
    e.k = 8;
    e.wpb = 8;
    e.threads = 512;
    e.blocks_per_cu = 2;
    e.symbol = L.name + "_xs";
    src << "extern \"C\" __global__ void __launch_bounds__(512) " << e.symbol << "(" << sig.str()
        << ", long long rows, long long cols, unsigned long long* status, unsigned* counter, unsigned ticket_base, "
        << "unsigned epoch, unp::waits wt) {\n" << ins.str() << "  unp::xscan_lookback<" << T << ", " << NI << ", "
        << f.op0 << ", " << ops << ", " << EX << ", " << RV << ", " << e.k << ", " << e.wpb << ", " << kScanStatusWords
        << (fixed ? ", true" : "") << ">(in, out, rows, cols, status, counter, ticket_base, epoch, wt);\n}\n";
  }
  L.entries.push_back(e);
  L.threads = e.threads;
  L.blocks_per_cu = e.blocks_per_cu;
  L.source = src.str();
  std::ostringstream j;
  j << "{\"backend\":\"hip\",\"target\":\"rocm:gfx950\",\"form\":\"scan\",\"dtype\":\"" << kind_name(f.dtype)
    << "\",\"op\":\"" << op_name(f.op0) << "\",\"exclusive\":" << EX << ",\"reverse\":" << RV << ",\"rank\":" << f.rank
    << ",\"axis\":" << axis << ",\"n_inputs\":" << NI << ",\"pre\":" << kir::write(rx.body)
    << ",\"post\":" << (rx.has_post ? kir::write(rx.post) : std::string("null"))
    << ",\"schedule\":\"" << (serial ? "serial" : fixed ? "fixed" : "device") << "\",\"params\":[";
  for (int k = 0; k < NI; ++k) j << "{\"name\":\"in" << k << "\",\"kind\":\"buffer\",\"role\":\"Read\"},";
  j << "{\"name\":\"out\",\"kind\":\"buffer\",\"role\":\"Write\"}";
  for (int d = 0; d < f.rank; ++d) j << ",{\"name\":\"n" << d << "\",\"kind\":\"scalar\",\"dtype\":\"I32\"}";
  j << "],\"launch\":{\"block\":[" << e.threads << ",1,1],\"grid\":\"cu_count*" << e.blocks_per_cu
    << "\",\"grid_policy\":\""
    << (serial ? "device-class constant; one lane per column of the inputs seen as A x S x B around the scanned axis"
               : "device-class constant; block tiles of 4096 positions taken by ticket, decoupled look-back")
    << "\"},\"entries\":[{\"symbol\":\"" << e.symbol << "\",\"when\":\"always\"}],\"workspace\":"
    << (serial ? std::string("null")
               : "{\"status\":\"tiles * " + std::to_string(kScanStatusWords * 8) +
                     " bytes, zeroed once\",\"counter\":4,\"stall\":4,\"host_state\":[\"epoch\",\"ticket_base\"]}")
    << ",\"compiler_args\":[\"--offload-arch=gfx950\",\"-O3\",\"-Xclang\",\"-target-feature\",\"-Xclang\",\"-packed-fp32-ops\"]"
    << ",\"fidelity_notes\":["
    << json_str(int_body ? "the pre evaluates at the element type by the total integer rule (Add/Sub/Mul wrap, a zero "
                           "divisor and MIN / -1 give the dividend, shift counts modulo the width) and the fold wraps at "
                           "the element type: every order gives the serial kernel's bits"
                : serial ? "the pre and the post evaluate in f64 and round once per statement, as the kernel evaluator runs "
                         "the lifted kernel; the fold in the serial lift's own order: bit-exact against the serial kernel"
                : fixed ? "the pre and the post evaluate in f64 and round once per statement; a Sum's prefixes are f64 "
                          "folds of the pre-mapped elements in an order the 4096-position block tiles fix (wave-local "
                          "scans; a tile's carry folds the totals of 64-tile groups, then the wave-tree prefix of its "
                          "group's earlier aggregates): the same bits on every launch, within the declared per-prefix "
                          "bound gamma_(n-1)*sum|v| + 1/2 ulp before the post; Max/Min exact except NaN payload and the "
                          "sign of a zero, which the tiling fixes too"
                        : "the pre and the post evaluate in f64 and round once per statement; a Sum's prefixes are f64 "
                          "folds of the pre-mapped elements in another order (wave-local scans and decoupled look-back), "
                          "within the declared per-prefix bound gamma_(n-1)*sum|v| + 1/2 ulp before the post, and not "
                          "reproducible run to run; Max/Min exact except NaN payload and the sign of a zero")
    << "]}";
  L.interface_json = j.str();
  return UNP_OK;
}

int32_t lower_form(const unp_form& f, Lowered& out, std::string& detail) {
  out = Lowered{};
  out.form = f;
  if (f.schedule != UNP_SCHEDULE_DEVICE && f.schedule != UNP_SCHEDULE_SERIAL && f.schedule != UNP_SCHEDULE_FIXED) {
    detail = "an unknown schedule";
    return UNP_UNSUPPORTED_SCHEDULE;
  }
  switch (f.kind) {
    case UNP_FORM_REDUCTION:
    case UNP_FORM_ROW_REDUCE2:
      return lower_reduction(f, out, detail);
    case UNP_FORM_SCAN:
      return lower_scan(f, out, detail);
    case UNP_FORM_GATHER:
      return lower_gather(f, out, detail);
    case UNP_FORM_DEQUANT4:
      return lower_dequant(f, out, detail);
    case UNP_FORM_DEQUANT_GEMM:
      return lower_dequant_gemm(f, out, detail);
    case UNP_FORM_ROW_REDUCE:
      detail = "a row reduction's expressions come only with its KernelFn (Backend::lower_kernel)";
      return UNP_UNSUPPORTED_KERNEL;
    case UNP_FORM_ELEMENTWISE:
      detail = "an elementwise op's body comes only with its KernelFn (Backend::lower_kernel)";
      return UNP_UNSUPPORTED_KERNEL;
    default:
      detail = "an unknown form";
      return UNP_UNSUPPORTED_KERNEL;
  }
}

// Backend::lower_variants for a form: the serial schedule (the cell's default: the sequential
// fold's bits) and the device schedule with its fidelity against it.  Forms whose schedules all
// give the same bits list one variant; the fused row fold, which has no serial schedule, lists
// its device schedule as its default.
int32_t form_variants(const unp_form& f, std::vector<unp_variant>& out, std::string& detail) {
  out.clear();
  unp_form dev = f, ser = f;
  dev.schedule = UNP_SCHEDULE_DEVICE;
  ser.schedule = UNP_SCHEDULE_SERIAL;
  Lowered L;
  const int32_t rc = lower_form(dev, L, detail);
  if (rc != UNP_OK) return rc;
  auto add = [&](const char* tag, int32_t fid, const unp_form& form, const std::string& note) {
    unp_variant v{};
    std::snprintf(v.tag, sizeof(v.tag), "%s", tag);
    v.fidelity = fid;
    v.form = form;
    std::snprintf(v.launch_note, sizeof(v.launch_note), "%s", note.c_str());
    out.push_back(v);
  };
  const bool fl = kind_is_float(f.dtype);
  if (f.kind == UNP_FORM_REDUCTION) {
    add("serial", UNP_BIT_IDENTICAL, ser, "one lane per output, the serial lift's order and accumulator");
    if (L.red_schedule != 'q') {
      // Order-free integer folds give the same bits in any order; a float fold's device order is
      // fixed for a device class but not the serial one (Sum/Mean round differently; Max/Min/
      // MaxNum/MinNum may keep another NaN payload or zero sign).
      add("device", fl ? UNP_DETERMINISTICALLY_DIVERGENT : UNP_BIT_IDENTICAL, dev,
          "cu_count x blocks_per_cu blocks; one launch (the full reduction and the split column "
          "reduction fold their partials in a last-ticket block)");
    }
    return UNP_OK;
  }
  if (f.kind == UNP_FORM_SCAN) {
    add("serial", UNP_BIT_IDENTICAL, ser, "one lane per column, the serial lift's order and accumulator");
    if (!L.serial_scan) {
      if (fl) {
        // The launch with the look-back's association fixed by the tiling (the default of a lifted
        // float scan): reproducible, in a different order from the serial fold.
        unp_form fix = f;
        fix.schedule = UNP_SCHEDULE_FIXED;
        add("fixed", UNP_DETERMINISTICALLY_DIVERGENT, fix,
            "persistent blocks drawing tile tickets, the look-back folding tile aggregates in groups of 64 "
            "tiles in a fixed association: the same bits every launch");
      }
      // The look-back carry's association depends on how far each look-back walked, which
      // depends on timing: a float result can differ from launch to launch.
      add("device", fl ? UNP_NONDETERMINISTIC : UNP_BIT_IDENTICAL, dev,
          "one persistent block per CU drawing tile tickets; decoupled look-back over a tile-status "
          "workspace tagged with a launch epoch");
    }
    return UNP_OK;
  }
  // The gather, the dequants and the fused row fold: one schedule.
  std::string note = "entries picked per launch by alignment and shape:";
  for (const Entry& e : L.entries) note += " " + e.symbol.substr(L.name.size());
  add("device", UNP_BIT_IDENTICAL, dev, note);
  return UNP_OK;
}

}  // namespace unp
