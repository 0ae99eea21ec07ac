// Internal declarations shared by the unpopped-hip host library's translation units.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/unpopped_hip.h"
#include "kernel_ir.hpp"

namespace unp {

// Element kinds the HIP forms move or compute (names as the reference's JSON spells them,
// crates/unpopped/src/text.rs:56-91).
const char* kind_name(int32_t kind);
int32_t kind_from_name(const std::string& s);  // -1 when unknown
size_t kind_bytes(int32_t kind);                // 0 for sub-byte and unknown kinds
bool kind_is_float(int32_t kind);
bool kind_is_int(int32_t kind);

// One entry point of a lowered kernel and when the executor picks it.
struct Entry {
  std::string symbol;
  int vec = 1;        // elements per lane-vector (reduce/scan), bytes per unit (gather)
  int k = 1;          // vectors per lane per tile (scan)
  int wpb = 1;        // waves per ticket group (scan)
  bool fast = false;  // the 16-byte-aligned path
  bool wide = false;  // reduction: the block-per-row schedule (long rows)
  int threads = 0;    // block size of this entry (0: the form's)
  int blocks_per_cu = 0;  // persistent blocks per CU of this entry (0: the form's)
  int cols = 0;           // output columns per block (dequant GEMM decode entries)
  // Reads and writes its buffers through storage-image strides (unp_hip_exec_launch_views with a
  // view that is not dense row-major); never picked for a pointer launch.
  bool strided = false;
};

// Scan tile status: words per tile (a 256-byte stride: the status of consecutive tiles, which
// every block probes at once, spreads over cache lines and memory channels).
constexpr int kScanStatusWords = 32;

// Reductions over more than kWideRow elements per row use the block-per-row schedule.
constexpr long long kWideRow = 32768;

// The reduced-axis mask of a reduction form (axes_mask, or reduced_from..rank-1 when it is 0)
// and its schedule class ('r', 'a', 'm' or 'g', as Lowered::red_schedule).
uint32_t reduction_mask(const unp_form& f);
char reduction_schedule(uint32_t mask, int32_t rank);

// The host image of the device's axes_desc (reduce_generic's argument, passed by value).
struct axes_desc_host {
  long long nk, nr;
  long long kext[8], kstr[8];
  long long rext[8], rstr[8];
  long long outs, count;
};

// Host images of the storage-image descriptors (red_view, scan_view, gather_view; passed by
// value): extents and signed element strides of the views, axes outermost first.
struct red_view_host {
  long long nk, nr;
  long long kext[8], kstr[8], kost[8];
  long long rext[8], rstr[8];
  long long outs, count;
};
struct scan_view_host {
  long long nc;
  long long cext[8], cin[8], cout[8];
  long long S, sin, sout;
  long long cols;
};
struct gather_view_host {
  long long rank, axis;
  long long ext[8], tstr[8], istr[8], ostr[8];
  long long outs;
};
struct gather_x_view_host {
  long long rank, axis;
  long long ext[8], ostr[8];
  long long istr[8][8];
  long long outs;
};

// An Access::RowReduce (crates/unpopped/src/ir.rs:2114-2125): the stages' pre expressions and
// folds, then the full-width epilogue, as ScalarExpr JSON over Input(k) and Reduced(t) leaves.
struct RowReduceSpec {
  int32_t dtype = 0;     // F32 or F64: the compute dtype of inputs, stages and output
  int32_t rank = 0;      // the reduced axis is the innermost; the output has the input's shape
  int32_t n_inputs = 0;
  std::vector<int32_t> ops;  // ReduceOp per stage
  std::vector<kir::J> pres;  // pre expression per stage
  kir::J epilogue;
};

// A reduction's pre-map body and fused post (the reduction lift's OpDef body and
// Access::Reduction post, kernel_lift.rs:807-831): `plain` when the body is Input(0) over one
// input and the post is the identity, which the plain reduction kernels lower.
struct ReductionExpr {
  bool plain = true;
  int32_t n_inputs = 1;
  kir::J body;  // ScalarExpr over Input(0..n_inputs)
  bool has_post = false;
  kir::J post;  // ScalarExpr over Reduced(0)
};

// A recognised gather beyond OpDef::gather (kernel_lift/gather.rs:35-101): n inputs, the index and
// the gathered data among them (form.data_slot), and an elementwise body over Input(0..n).  plain:
// the two-input identity gather the row kernels move.
struct GatherExpr {
  bool plain = true;
  int32_t n_inputs = 2;
  int32_t index_slot = 1;
  kir::J body;  // ScalarExpr over Input(k)
};

// A recognised Access::Elementwise lift (kernel_lift.rs:96-130): n inputs read at the output
// coordinate (input k through the axis permutation perms[k] when it is not empty: iteration axis d
// reads the input's axis perms[k][d], kernel_lift.rs:315-324) and a body over Input(0..n) stored
// at the output coordinate.
struct ElementwiseExpr {
  int32_t n_inputs = 1;
  kir::J body;  // ScalarExpr over Input(k)
  std::vector<std::vector<int32_t>> perms;
  bool permuted() const {
    for (const auto& p : perms)
      for (size_t d = 0; d < p.size(); ++d)
        if (p[d] != (int32_t)d) return true;
    return false;
  }
};

// A lowered form: what the executor needs to launch it.
struct Lowered {
  unp_form form{};
  std::string name;
  std::string source;
  std::string interface_json;
  std::vector<Entry> entries;
  bool reduce_all = false;  // a reduction with no kept axis
  // A reduction's schedule, from the shape of its reduced-axis set once adjacent axes of a
  // kind are merged: 'r' kept then reduced (rows), 'a' all reduced, 'm' one reduced run with
  // kept axes after it (A x R x B), 'g' anything else.
  char red_schedule = 'r';
  uint32_t axes_mask = 0;  // the reduced axes, bit d = axis d
  int threads = 256;
  int blocks_per_cu = 8;
  // A scan in the serial lift's own order (a non-innermost axis, or a float Prod): the scanned
  // axis, and the input seen as A x S x B around it.
  bool serial_scan = false;
  int32_t scan_axis = 0;
  RowReduceSpec rr;  // UNP_FORM_ROW_REDUCE only
  ReductionExpr rx;  // UNP_FORM_REDUCTION and UNP_FORM_SCAN: the pre-map body and the post
  GatherExpr gx;     // UNP_FORM_GATHER: the inputs and body
  ElementwiseExpr ew;  // UNP_FORM_ELEMENTWISE: the inputs, their permutations and the body
};

// Emit the HIP source and interface for `f`; on refusal returns a nonzero unp_status and
// fills `detail`.
int32_t lower_form(const unp_form& f, Lowered& out, std::string& detail);
// Backend::lower_variants for a form: its schedules with their fidelity, the default first.
int32_t form_variants(const unp_form& f, std::vector<unp_variant>& out, std::string& detail);
// A recognised reduction with its body and post (the plain ones go to lower_form).
int32_t lower_reduction_x(const unp_form& f, const ReductionExpr& rx, Lowered& out, std::string& detail);
int32_t lower_scan_x(const unp_form& f, const ReductionExpr& rx, Lowered& out, std::string& detail);
// A recognised gather with more inputs or a body (the plain ones go to lower_form).
int32_t lower_gather_x(const unp_form& f, const GatherExpr& gx, Lowered& out, std::string& detail);
// The same for a recognised Access::RowReduce.
int32_t lower_row_reduce(const RowReduceSpec& spec, Lowered& out, std::string& detail);
// A recognised Access::Elementwise (its body comes only with the KernelFn).
int32_t lower_elementwise(const unp_form& f, const ElementwiseExpr& ew, Lowered& out, std::string& detail);

// Backend::lower_kernel's recognizer (lifts.cpp): the form a KernelFn's JSON is, or a refusal.
// A recognised kernel: the form to lower, the lift it matched, and the kernel's name, declared
// launch and parameters (the core half of its interface).
struct Recognized {
  unp_form form{};
  RowReduceSpec rr;  // UNP_FORM_ROW_REDUCE only
  ReductionExpr rx;  // UNP_FORM_REDUCTION and UNP_FORM_SCAN
  GatherExpr gx;     // UNP_FORM_GATHER only
  ElementwiseExpr ew;  // UNP_FORM_ELEMENTWISE only
  std::string lift;
  kir::J launch;
  kir::J params;
  std::string name;
};
int32_t recognize_kernel(const std::string& text, Recognized& out, std::string& why);

// hipRTC for gfx950, with an in-process compile-once cache keyed by source text.
int32_t compile_source(const std::string& source, const std::string& entry, uint32_t max_ms,
                       std::vector<uint8_t>& code, std::string& log);

// FNV-1a 64 (crates/unpopped/src/revision.rs).
uint64_t fnv1a64(const std::string& s);

void set_error(unp_error* err, int32_t code, const std::string& detail);

// A caller-provided device region that a no-allocation launch carves its workspaces from.
struct Scratch {
  void* base;
  size_t cap;
};
// Zero `bytes` (a multiple of 16) at the device address `base` with a kernel on `stream`
// (scratch.hip): the static scratch's per-call clear, a kernel node under graph capture.
int32_t scratch_clear(void* base, size_t bytes, void* stream, unp_error* err);

// Staged storage images (views.hip): the dense bytes a view of `bits`-bit elements packs into, the
// pack of an input view into `dst` (row-major over its shape), and the unpack of a dense output into
// its view, each as kernels on `stream`.
size_t view_stage_bytes(const unp_view& v, int bits);
int32_t view_stage_in(const unp_view& v, int bits, void* dst, void* stream, unp_error* err);
int32_t view_stage_out(const void* src, const unp_view& v, int bits, void* stream, unp_error* err);
// unp_hip_exec_launch with every workspace taken from [scratch, scratch + cap) and cleared on the
// launch stream first: it calls no allocator, and refuses a launch whose workspace does not fit
// with UNP_INVALID_ARGUMENT before anything runs.
int32_t exec_launch_in(unp_exec* x, const unp_arg* args, size_t nargs, void* stream, void* scratch, size_t cap,
                       unp_error* err);

}  // namespace unp

struct unp_generated {
  unp::Lowered l;
};
