// The backend's C entry points, the HIP runtime FFI and the prepared-kernel executor.
//
// The executor is the consumer-side launch layer the reference leaves out by rule
// (docs/PATENT-SWEEP.md:265-272): it compiles a lowered kernel's source once, loads it with
// hipModuleLoadData, picks the entry point whose alignment preconditions the arguments meet,
// owns the scan's tile-status and the full reduction's partials workspaces, and launches with
// hipModuleLaunchKernel.
//
// Launch geometry follows the reference's rule that no block, grid or thread count is derived
// from a loop bound (docs/PATENT-SWEEP.md:269): every reduction, scan, gather, row-reduce and
// dequant launch takes a device-class grid (cu_count times the entry's blocks per CU) and its
// blocks stride over the work, the surplus exiting.  The work decomposition itself (the column
// reduction's chunks of the reduced axis, the scan's tiles) is sized from the extents; it sets
// how many items the fixed grid strides over, not how many blocks run.  The dequantizing GEMM's
// decode, MFMA and prep kernels do the same over their (row tile, split of K, column tile), tile
// and (group, column slab) items.  One entry departs from the rule: the streaming entry launches a
// block per item (an item loop around its LDS pipeline made it spill).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "kernel_ir.hpp"
#include "unp_internal.hpp"

// libamdhip64's launch with kernel-timestamp events (declared in hip/hip_ext.h, whose C++ helpers
// need the HIP compiler; this file is compiled by the host compiler).
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                               uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                               uint32_t localWorkSizeY, uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void** kernelParams, void** extra,
                                               hipEvent_t startEvent, hipEvent_t stopEvent, uint32_t flags);

using unp::set_error;

namespace {

int32_t hip_fail(unp_error* err, const char* what, hipError_t e) {
  set_error(err, UNP_HIP_ERROR, std::string(what) + ": " + hipGetErrorString(e));
  return UNP_HIP_ERROR;
}

bool valid_target(const char* t) {
  if (!t) return false;
  int colons = 0;
  size_t n = std::strlen(t), at = 0;
  for (size_t i = 0; i < n; ++i) {
    const unsigned char c = (unsigned char)t[i];
    if (c == ':') {
      ++colons;
      at = i;
    }
    if (c <= 0x20 || c >= 0x7f || c == '|' || c == ';' || c == '/') return false;
  }
  return colons == 1 && at > 0 && at + 1 < n;
}

// How long one wait of a kernel for another block may last before the kernel gives up on it
// (unp_hip_exec_set_wait_limit): a wait that the hardware serves takes microseconds.
constexpr uint32_t kDefaultWaitUs = 1000000;

uint32_t wait_ticks_for(int khz, uint32_t us) {
  const unsigned long long t = (unsigned long long)khz * us / 1000ull;
  return t > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)t;
}

// The device's `waits` kernel argument: the stall word and the bound in wall-clock ticks.
struct waits_host {
  uint32_t* stall;
  uint32_t ticks;
  uint32_t pad;
};
static_assert(sizeof(waits_host) == 16, "waits_host mirrors the device's waits");

}  // namespace

struct unp_module {
  hipModule_t m = nullptr;
};
struct unp_function {
  hipFunction_t f = nullptr;
};
struct unp_event {
  hipEvent_t e = nullptr;
};

struct unp_exec {
  unp::Lowered l;
  hipModule_t mod = nullptr;
  std::vector<hipFunction_t> fns;
  // Blocks of each entry that one CU holds at once, by its registers and LDS (0: not asked).
  std::vector<int> resident;
  int device = 0;
  int cu_count = 0;
  void* ws = nullptr;  // scan: tile status words; full reduction: block partials
  size_t ws_bytes = 0;
  uint32_t* counter = nullptr;
  uint32_t* counters = nullptr;  // reduce_mid: one ticket counter per column strip, left zero
  size_t n_counters = 0;
  uint32_t epoch = 0;
  uint32_t ticket_base = 0;
  // Bounded waits: the word a kernel that gave up waiting counts into, read and cleared by
  // unp_hip_exec_check, and the bound in ticks of the device's wall clock (wall_clock_khz kHz).
  uint32_t* stall = nullptr;
  uint32_t wait_ticks = 0;
  int wall_clock_khz = 0;
  // Set for the duration of a no-allocation launch: every workspace is carved from this region
  // (cleared first) instead of the executor's own allocations.
  const unp::Scratch* fixed = nullptr;
  // Kernel timing for reports: the first kernel of a launch records t_start at its beginning and
  // every kernel records t_stop at its end (their own dispatch timestamps).
  hipEvent_t t_start = nullptr, t_stop = nullptr;
  bool t_first = false;
  uint32_t grid[3] = {0, 0, 0};
  uint32_t block[3] = {0, 0, 0};
  std::string last_entry;
  // Dense copies of staged storage images, one per buffer parameter (grown on demand).
  std::vector<void*> stage;
  std::vector<size_t> stage_cap;
};

extern "C" {

// ---------------------------------------------------------------------------------------
// Backend seam
// ---------------------------------------------------------------------------------------

const char* unp_hip_name(void) { return "hip"; }
const char* unp_hip_provider(void) { return "unpopped-hip"; }
// Integer Div, Shl, Shr and ConstInt are spelled by the total rule (unp::xi in the device library).
int32_t unp_hip_total_integer_ops(void) { return 1; }

int32_t unp_hip_supports_dtype(int32_t kind, const char* target) {
  if (!valid_target(target)) return UNP_UNSUPPORTED;
  const std::string t(target);
  if (t.rfind("rocm:gfx950", 0) != 0) return UNP_UNSUPPORTED;
  switch (kind) {
    case UNP_F16: case UNP_BF16: case UNP_F32: case UNP_F32_STRICT: case UNP_F64:
    case UNP_I8: case UNP_I16: case UNP_U8: case UNP_U16: case UNP_I32: case UNP_I64:
    case UNP_BOOL: case UNP_U32: case UNP_U64: case UNP_I4: case UNP_U4:
      return UNP_SUPPORTED;
    default:
      return UNP_UNSUPPORTED;
  }
}

int32_t unp_hip_lower_form(const unp_form* form, unp_generated** out, unp_error* err) {
  if (out) *out = nullptr;
  if (!form || !out) {
    set_error(err, UNP_INVALID_ARGUMENT, "null form or output");
    return UNP_INVALID_ARGUMENT;
  }
  auto* g = new unp_generated();
  std::string why;
  const int32_t rc = unp::lower_form(*form, g->l, why);
  if (rc != UNP_OK) {
    delete g;
    set_error(err, rc, why);
    return rc;
  }
  set_error(err, UNP_OK, "");
  *out = g;
  return UNP_OK;
}

int32_t unp_hip_form_variants(const unp_form* form, unp_variant* out, size_t cap, size_t* count, unp_error* err) {
  if (count) *count = 0;
  if (!form || !count || (cap && !out)) {
    set_error(err, UNP_INVALID_ARGUMENT, "null form, output or count");
    return UNP_INVALID_ARGUMENT;
  }
  std::vector<unp_variant> vs;
  std::string why;
  const int32_t rc = unp::form_variants(*form, vs, why);
  if (rc != UNP_OK) {
    set_error(err, rc, why);
    return rc;
  }
  for (size_t i = 0; i < vs.size() && i < cap; ++i) out[i] = vs[i];
  *count = vs.size();
  set_error(err, UNP_OK, "");
  return UNP_OK;
}

int32_t unp_hip_lower_kernel(const char* kernel_json, unp_generated** out, unp_error* err) {
  if (out) *out = nullptr;
  if (!kernel_json || !out) {
    set_error(err, UNP_INVALID_ARGUMENT, "null kernel or output");
    return UNP_INVALID_ARGUMENT;
  }
  unp::Recognized rec;
  std::string why;
  int32_t rc = unp::recognize_kernel(kernel_json, rec, why);
  if (rc != UNP_OK) {
    set_error(err, rc, why);
    return rc;
  }
  // A lifted float scan lowers the fixed schedule: its carries fold in an order the tiling
  // fixes, so every launch gives the same bits, as the reference's launched scan lift promises
  // (kernel_lift/scan_launched.rs:22-27).  The device schedule's look-back, whose float
  // association depends on timing, is only a Nondeterministic variant (unp_hip_form_variants).
  if (rec.form.kind == UNP_FORM_SCAN && unp::kind_is_float(rec.form.dtype) && rec.form.schedule == UNP_SCHEDULE_DEVICE)
    rec.form.schedule = UNP_SCHEDULE_FIXED;
  auto* g = new unp_generated();
  if (rec.form.kind == UNP_FORM_ROW_REDUCE || rec.form.kind == UNP_FORM_ELEMENTWISE) {
    // A row reduction or elementwise op whose expressions hold a node this backend cannot spell
    // is an UnsupportedOp (backend.rs:398-403), one at a dtype it has no spelling for an
    // UnsupportedDtype, its other refusals an UnsupportedKernel.
    rc = rec.form.kind == UNP_FORM_ROW_REDUCE ? unp::lower_row_reduce(rec.rr, g->l, why)
                                              : unp::lower_elementwise(rec.form, rec.ew, g->l, why);
    if (rc != UNP_OK) {
      delete g;
      if (rc != UNP_UNSUPPORTED_OP && rc != UNP_UNSUPPORTED_DTYPE) rc = UNP_UNSUPPORTED_KERNEL;
      set_error(err, rc, why);
      return rc;
    }
  } else {
    rc = rec.form.kind == UNP_FORM_REDUCTION                       ? unp::lower_reduction_x(rec.form, rec.rx, g->l, why)
         : rec.form.kind == UNP_FORM_SCAN                          ? unp::lower_scan_x(rec.form, rec.rx, g->l, why)
         : (rec.form.kind == UNP_FORM_GATHER && !rec.gx.plain) ? unp::lower_gather_x(rec.form, rec.gx, g->l, why)
                                                               : unp::lower_form(rec.form, g->l, why);
    if (rc != UNP_OK) {
      delete g;
      // A recognised lift whose form this backend has no kernel for is a refusal of the kernel.
      set_error(err, UNP_UNSUPPORTED_KERNEL, why);
      return UNP_UNSUPPORTED_KERNEL;
    }
  }
  // The interface's core half (KernelInterface::of, kernel_interface.rs:237-262): the kernel's
  // declared launch and parameters, beside the emitter half the form wrote.
  std::string& j = g->l.interface_json;
  j.pop_back();
  j += ",\"kernel\":" + unp::kir::write(unp::kir::J::str(rec.name)) + ",\"lift\":\"" + rec.lift +
       "\",\"declared_launch\":" + unp::kir::write(rec.launch) + ",\"kernel_params\":" + unp::kir::write(rec.params) +
       "}";
  set_error(err, UNP_OK, "");
  *out = g;
  return UNP_OK;
}

const char* unp_generated_name(const unp_generated* g) { return g ? g->l.name.c_str() : nullptr; }
const char* unp_generated_source(const unp_generated* g) { return g ? g->l.source.c_str() : nullptr; }
const char* unp_generated_interface_json(const unp_generated* g) {
  return g ? g->l.interface_json.c_str() : nullptr;
}
uint64_t unp_generated_revision_hash(const unp_generated* g) { return g ? unp::fnv1a64(g->l.source) : 0; }
void unp_generated_free(unp_generated* g) { delete g; }

// ---------------------------------------------------------------------------------------
// HIP runtime FFI
// ---------------------------------------------------------------------------------------

int32_t unp_hip_device_count(int32_t* count) {
  int n = 0;
  const hipError_t e = hipGetDeviceCount(&n);
  if (count) *count = (e == hipSuccess) ? n : 0;
  return e == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}

int32_t unp_hip_set_device(int32_t device) { return hipSetDevice(device) == hipSuccess ? UNP_OK : UNP_HIP_ERROR; }

int32_t unp_hip_device_info(char* arch, size_t arch_len, int32_t* cu_count) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return UNP_HIP_ERROR;
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess) return UNP_HIP_ERROR;
  if (arch && arch_len) std::snprintf(arch, arch_len, "%s", p.gcnArchName);
  if (cu_count) *cu_count = p.multiProcessorCount;
  return UNP_OK;
}

int32_t unp_hip_module_load(const uint8_t* image, size_t len, unp_module** out, unp_error* err) {
  if (out) *out = nullptr;
  if (!image || !len || !out) {
    set_error(err, UNP_INVALID_ARGUMENT, "empty code object");
    return UNP_INVALID_ARGUMENT;
  }
  hipModule_t m = nullptr;
  const hipError_t e = hipModuleLoadData(&m, image);
  if (e != hipSuccess) return hip_fail(err, "hipModuleLoadData", e);
  *out = new unp_module{m};
  return UNP_OK;
}

int32_t unp_hip_module_unload(unp_module* m) {
  if (!m) return UNP_OK;
  const hipError_t e = hipModuleUnload(m->m);
  delete m;
  return e == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}

int32_t unp_hip_get_function(unp_module* m, const char* name, unp_function** out, unp_error* err) {
  if (out) *out = nullptr;
  if (!m || !name || !out) {
    set_error(err, UNP_INVALID_ARGUMENT, "null module, name or output");
    return UNP_INVALID_ARGUMENT;
  }
  hipFunction_t f = nullptr;
  const hipError_t e = hipModuleGetFunction(&f, m->m, name);
  if (e != hipSuccess) return hip_fail(err, "hipModuleGetFunction", e);
  *out = new unp_function{f};
  return UNP_OK;
}

int32_t unp_hip_launch(unp_function* f, const uint32_t grid[3], const uint32_t block[3], uint32_t shared_bytes,
                       void* stream, const void* kernarg, size_t kernarg_size, unp_error* err) {
  if (!f || !grid || !block || (kernarg_size && !kernarg)) {
    set_error(err, UNP_INVALID_ARGUMENT, "null function, geometry or argument block");
    return UNP_INVALID_ARGUMENT;
  }
  size_t size = kernarg_size;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(kernarg), HIP_LAUNCH_PARAM_BUFFER_SIZE,
                    &size, HIP_LAUNCH_PARAM_END};
  const hipError_t e = hipModuleLaunchKernel(f->f, grid[0], grid[1], grid[2], block[0], block[1], block[2],
                                             shared_bytes, (hipStream_t)stream, nullptr, config);
  if (e != hipSuccess) return hip_fail(err, "hipModuleLaunchKernel", e);
  return UNP_OK;
}

int32_t unp_hip_launch_timed(unp_function* f, const uint32_t grid[3], const uint32_t block[3], uint32_t shared_bytes,
                             void* stream, const void* kernarg, size_t kernarg_size, unp_event* start, unp_event* stop,
                             unp_error* err) {
  if (!f || !grid || !block || (kernarg_size && !kernarg)) {
    set_error(err, UNP_INVALID_ARGUMENT, "null function, geometry or argument block");
    return UNP_INVALID_ARGUMENT;
  }
  // hipExtModuleLaunchKernel takes work-items, not blocks.
  uint32_t items[3];
  for (int d = 0; d < 3; ++d) {
    if ((uint64_t)grid[d] * block[d] > 0xFFFFFFFFull) {
      set_error(err, UNP_INVALID_ARGUMENT, "a timed launch takes at most 2^32 - 1 work-items per dimension");
      return UNP_INVALID_ARGUMENT;
    }
    items[d] = grid[d] * block[d];
  }
  size_t size = kernarg_size;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(kernarg), HIP_LAUNCH_PARAM_BUFFER_SIZE,
                    &size, HIP_LAUNCH_PARAM_END};
  const hipError_t e = hipExtModuleLaunchKernel(f->f, items[0], items[1], items[2], block[0], block[1], block[2],
                                                shared_bytes, (hipStream_t)stream, nullptr, config,
                                                start ? start->e : nullptr, stop ? stop->e : nullptr, 0);
  if (e != hipSuccess) return hip_fail(err, "hipExtModuleLaunchKernel", e);
  return UNP_OK;
}

int32_t unp_hip_malloc(void** p, size_t bytes) {
  if (!p) return UNP_INVALID_ARGUMENT;
  *p = nullptr;
  return hipMalloc(p, bytes ? bytes : 1) == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}
int32_t unp_hip_free(void* p) { return hipFree(p) == hipSuccess ? UNP_OK : UNP_HIP_ERROR; }
int32_t unp_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}
int32_t unp_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost) == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}
int32_t unp_hip_memset(void* p, int32_t value, size_t bytes) {
  return hipMemset(p, value, bytes) == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}
int32_t unp_hip_synchronize(void) { return hipDeviceSynchronize() == hipSuccess ? UNP_OK : UNP_HIP_ERROR; }

int32_t unp_hip_event_create(unp_event** e) {
  if (!e) return UNP_INVALID_ARGUMENT;
  hipEvent_t h = nullptr;
  if (hipEventCreate(&h) != hipSuccess) return UNP_HIP_ERROR;
  *e = new unp_event{h};
  return UNP_OK;
}
int32_t unp_hip_event_destroy(unp_event* e) {
  if (!e) return UNP_OK;
  const hipError_t r = hipEventDestroy(e->e);
  delete e;
  return r == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}
int32_t unp_hip_event_record(unp_event* e, void* stream) {
  if (!e) return UNP_INVALID_ARGUMENT;
  return hipEventRecord(e->e, (hipStream_t)stream) == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}
int32_t unp_hip_event_synchronize(unp_event* e) {
  if (!e) return UNP_INVALID_ARGUMENT;
  return hipEventSynchronize(e->e) == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}
int32_t unp_hip_event_elapsed_ms(unp_event* start, unp_event* stop, float* ms) {
  if (!start || !stop || !ms) return UNP_INVALID_ARGUMENT;
  return hipEventElapsedTime(ms, start->e, stop->e) == hipSuccess ? UNP_OK : UNP_HIP_ERROR;
}

// ---------------------------------------------------------------------------------------
// Prepared kernels
// ---------------------------------------------------------------------------------------

int32_t unp_hip_exec_create(const unp_generated* g, unp_exec** out, unp_error* err) {
  if (out) *out = nullptr;
  if (!g || !out) {
    set_error(err, UNP_INVALID_ARGUMENT, "null kernel or output");
    return UNP_INVALID_ARGUMENT;
  }
  auto* x = new unp_exec();
  x->l = g->l;
  if (hipGetDevice(&x->device) != hipSuccess) {
    delete x;
    set_error(err, UNP_HIP_ERROR, "hipGetDevice failed (no HIP device)");
    return UNP_HIP_ERROR;
  }
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, x->device);
  if (e != hipSuccess) {
    delete x;
    return hip_fail(err, "hipGetDeviceProperties", e);
  }
  x->cu_count = p.multiProcessorCount;
  e = hipDeviceGetAttribute(&x->wall_clock_khz, hipDeviceAttributeWallClockRate, x->device);
  if (e != hipSuccess || x->wall_clock_khz <= 0) {
    delete x;
    return hip_fail(err, "hipDeviceGetAttribute(wall clock rate)", e != hipSuccess ? e : hipErrorInvalidValue);
  }
  x->wait_ticks = wait_ticks_for(x->wall_clock_khz, kDefaultWaitUs);
  e = hipMalloc((void**)&x->stall, sizeof(uint32_t));
  if (e == hipSuccess) e = hipMemset(x->stall, 0, sizeof(uint32_t));
  if (e != hipSuccess) {
    if (x->stall) hipFree(x->stall);
    delete x;
    return hip_fail(err, "hipMalloc(stall word)", e);
  }
  std::vector<uint8_t> code;
  std::string log;
  const int32_t rc = unp::compile_source(x->l.source, x->l.name, 0, code, log);
  if (rc != UNP_OK) {
    unp_hip_exec_destroy(x);
    set_error(err, rc, log);
    return rc;
  }
  e = hipModuleLoadData(&x->mod, code.data());
  if (e != hipSuccess) {
    x->mod = nullptr;
    unp_hip_exec_destroy(x);
    return hip_fail(err, "hipModuleLoadData", e);
  }
  for (const auto& en : x->l.entries) {
    hipFunction_t f = nullptr;
    e = hipModuleGetFunction(&f, x->mod, en.symbol.c_str());
    if (e != hipSuccess) {
      unp_hip_exec_destroy(x);
      return hip_fail(err, ("hipModuleGetFunction " + en.symbol).c_str(), e);
    }
    x->fns.push_back(f);
    int per_cu = 0;
    if (x->l.form.kind == UNP_FORM_ROW_REDUCE &&
        hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, en.threads > 0 ? en.threads : x->l.threads, 0) !=
            hipSuccess)
      per_cu = 0;
    x->resident.push_back(per_cu);
  }
  set_error(err, UNP_OK, "");
  *out = x;
  return UNP_OK;
}

void unp_hip_exec_destroy(unp_exec* x) {
  if (!x) return;
  if (x->ws) hipFree(x->ws);
  if (x->counter) hipFree(x->counter);
  if (x->counters) hipFree(x->counters);
  if (x->stall) hipFree(x->stall);
  for (void* p : x->stage)
    if (p) hipFree(p);
  if (x->mod) hipModuleUnload(x->mod);
  delete x;
}

int32_t unp_hip_exec_set_wait_limit(unp_exec* x, uint32_t wait_us) {
  if (!x) return UNP_INVALID_ARGUMENT;
  x->wait_ticks = wait_ticks_for(x->wall_clock_khz, wait_us);
  return UNP_OK;
}

int32_t unp_hip_exec_check(unp_exec* x, unp_error* err) {
  if (!x) {
    set_error(err, UNP_INVALID_ARGUMENT, "null executor");
    return UNP_INVALID_ARGUMENT;
  }
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(err, "hipDeviceSynchronize", e);
  uint32_t n = 0;
  e = hipMemcpy(&n, x->stall, sizeof n, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(err, "hipMemcpy(stall word)", e);
  if (n == 0) {
    set_error(err, UNP_OK, "");
    return UNP_OK;
  }
  e = hipMemset(x->stall, 0, sizeof n);
  if (e != hipSuccess) return hip_fail(err, "hipMemset(stall word)", e);
  set_error(err, UNP_STALLED,
            std::to_string(n) + " wait(s) in launches of `" + x->l.name + "` gave up after " +
                std::to_string((unsigned long long)x->wait_ticks * 1000ull / (unsigned long long)x->wall_clock_khz) +
                " us without the block they waited for; those launches' outputs are not valid");
  return UNP_STALLED;
}

int32_t unp_hip_exec_set_timing(unp_exec* x, unp_event* start, unp_event* stop) {
  if (!x || (start == nullptr) != (stop == nullptr)) return UNP_INVALID_ARGUMENT;
  x->t_start = start ? start->e : nullptr;
  x->t_stop = stop ? stop->e : nullptr;
  return UNP_OK;
}

int32_t unp_hip_exec_last_launch(const unp_exec* x, uint32_t grid[3], uint32_t block[3], char* entry,
                                 size_t entry_len) {
  if (!x) return UNP_INVALID_ARGUMENT;
  for (int i = 0; i < 3; ++i) {
    if (grid) grid[i] = x->grid[i];
    if (block) block[i] = x->block[i];
  }
  if (entry && entry_len) std::snprintf(entry, entry_len, "%s", x->last_entry.c_str());
  return UNP_OK;
}

}  // extern "C"

namespace {

bool aligned16(uint64_t p) { return (p & 15u) == 0; }

// Reads the KernelFn-ordered arguments: `nbuf` buffers then `nscal` scalars.
struct Args {
  std::vector<uint64_t> buf;
  std::vector<int64_t> ext;
};

int32_t take_args(const unp_arg* a, size_t n, size_t nbuf, size_t nscal, Args& out, unp_error* err) {
  if (n != nbuf + nscal || (n && !a)) {
    set_error(err, UNP_INVALID_ARGUMENT,
              "expected " + std::to_string(nbuf) + " buffers and " + std::to_string(nscal) + " scalars, got " +
                  std::to_string(n) + " arguments");
    return UNP_INVALID_ARGUMENT;
  }
  for (size_t i = 0; i < n; ++i) {
    const bool want_buf = i < nbuf;
    if ((a[i].is_buffer != 0) != want_buf) {
      set_error(err, UNP_INVALID_ARGUMENT, "argument " + std::to_string(i) + (want_buf ? " must be a buffer" : " must be a scalar"));
      return UNP_INVALID_ARGUMENT;
    }
    if (want_buf) out.buf.push_back(a[i].value);
    else out.ext.push_back((int64_t)a[i].value);
  }
  return UNP_OK;
}

// The reference's extents are I32 scalars: read the low 32 bits as signed.
int32_t extents_i32(Args& A, size_t count, unp_error* err) {
  for (size_t i = 0; i < count; ++i) {
    const int64_t v = (int64_t)(int32_t)(uint32_t)(uint64_t)A.ext[i];
    if (v < 0) {
      set_error(err, UNP_INVALID_ARGUMENT, "extent n" + std::to_string(i) + " is negative");
      return UNP_INVALID_ARGUMENT;
    }
    A.ext[i] = v;
  }
  return UNP_OK;
}

int32_t need_buffers(const Args& A, bool any_elements, unp_error* err) {
  if (!any_elements) return UNP_OK;
  for (size_t i = 0; i < A.buf.size(); ++i)
    if (A.buf[i] == 0) {
      set_error(err, UNP_INVALID_ARGUMENT, "buffer argument " + std::to_string(i) + " is null");
      return UNP_INVALID_ARGUMENT;
    }
  return UNP_OK;
}

int32_t ensure_ws(unp_exec* x, size_t bytes, bool need_counter, unp_error* err) {
  if (need_counter && !x->counter) {
    hipError_t e = hipMalloc((void**)&x->counter, sizeof(uint32_t));
    if (e != hipSuccess) return hip_fail(err, "hipMalloc(counter)", e);
    e = hipMemset(x->counter, 0, sizeof(uint32_t));
    if (e != hipSuccess) return hip_fail(err, "hipMemset(counter)", e);
  }
  if (bytes > x->ws_bytes) {
    if (x->ws) {
      hipFree(x->ws);
      x->ws = nullptr;
      x->ws_bytes = 0;
    }
    hipError_t e = hipMalloc(&x->ws, bytes);
    if (e != hipSuccess) return hip_fail(err, "hipMalloc(workspace)", e);
    e = hipMemset(x->ws, 0, bytes);
    if (e != hipSuccess) return hip_fail(err, "hipMemset(workspace)", e);
    x->ws_bytes = bytes;
  }
  return UNP_OK;
}

// The workspaces of one launch: the executor's own allocations, or, in a no-allocation launch,
// 256-byte-aligned pieces of the caller's scratch region (a ticket counter, then the counters,
// then the workspace), cleared on the launch stream before the kernel runs.
struct Ws {
  void* ws = nullptr;
  uint32_t* counter = nullptr;
  uint32_t* counters = nullptr;
};

int32_t ensure_counters(unp_exec* x, size_t n, unp_error* err);

int32_t workspace(unp_exec* x, size_t bytes, bool need_counter, size_t n_counters, hipStream_t s, Ws& w,
                  unp_error* err) {
  if (x->fixed) {
    const auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    const size_t need = (need_counter ? 256 : 0) + up(n_counters * sizeof(uint32_t)) + up(bytes);
    // The last 256 bytes stay unused, so no piece ends at the region's very end.
    if (x->fixed->cap < 256 || need > x->fixed->cap - 256) {
      set_error(err, UNP_INVALID_ARGUMENT,
                "this launch needs " + std::to_string(need) + " bytes of workspace; the static scratch holds " +
                    std::to_string(x->fixed->cap) + " (" + std::to_string(x->fixed->cap - 256) + " usable)");
      return UNP_INVALID_ARGUMENT;
    }
    uint8_t* p = static_cast<uint8_t*>(x->fixed->base);
    if (need_counter) {
      w.counter = reinterpret_cast<uint32_t*>(p);
      p += 256;
    }
    if (n_counters) {
      w.counters = reinterpret_cast<uint32_t*>(p);
      p += up(n_counters * sizeof(uint32_t));
    }
    if (bytes) w.ws = p;
    // A kernel, not hipMemsetAsync: a call under graph capture then records no memset node.
    if (need) return unp::scratch_clear(x->fixed->base, need, s, err);
    return UNP_OK;
  }
  int32_t rc = ensure_ws(x, bytes, need_counter, err);
  if (rc == UNP_OK && n_counters) rc = ensure_counters(x, n_counters, err);
  if (rc != UNP_OK) return rc;
  w.ws = x->ws;
  w.counter = x->counter;
  w.counters = x->counters;
  return UNP_OK;
}

// The epoch of a launch whose kernels tag their hand-off words (scan tile status, reduction
// partials): 1 in a no-allocation launch, whose scratch was just cleared; else the executor's
// next, after clearing its words when the 31-bit epoch would wrap (the scan's status words keep
// 31 bits of it), so that no word is ever taken for one an earlier launch wrote.
int32_t next_epoch(unp_exec* x, hipStream_t s, uint32_t& ep, unp_error* err) {
  if (x->fixed) {
    ep = 1;
    return UNP_OK;
  }
  if (x->epoch == 0x7fffffffu) {
    const hipError_t e = hipMemsetAsync(x->ws, 0, x->ws_bytes, s);
    if (e != hipSuccess) return hip_fail(err, "hipMemsetAsync(tagged words)", e);
    x->epoch = 0;
  }
  ep = ++x->epoch;  // the words start zeroed, so epoch 1 is never seen before the first launch
  return UNP_OK;
}

waits_host waits_of(const unp_exec* x) { return waits_host{x->stall, x->wait_ticks, 0}; }

// The kept and the reduced axes of a row-major input with their element strides, outermost
// first, adjacent axes of a kind merged (a merged run's stride is its innermost axis's).
void fill_axes_desc(const std::vector<int64_t>& ext, int32_t rank, uint32_t mask, unp::axes_desc_host& d) {
  long long stride = 1;
  std::vector<long long> str((size_t)rank);
  for (int32_t k = rank - 1; k >= 0; --k) {
    str[(size_t)k] = stride;
    stride *= ext[(size_t)k];
  }
  for (int32_t k = 0; k < rank;) {
    const bool red = (mask >> k) & 1u;
    long long e_ = 1;
    int32_t e = k;
    while (e < rank && (((mask >> e) & 1u) != 0) == red) e_ *= ext[(size_t)e++];
    const long long st = str[(size_t)(e - 1)];
    if (red) {
      d.rext[d.nr] = e_;
      d.rstr[d.nr++] = st;
    } else {
      d.kext[d.nk] = e_;
      d.kstr[d.nk++] = st;
    }
    k = e;
  }
}

// Appends axis (e, is, os) to a descriptor's list, merged into the previous axis when the two
// walk storage as one (the previous stride is this axis's extent times its stride, in every
// buffer); axes of extent 1 add nothing.
template <int NS>
void add_axis(long long* ext, long long* const (&str)[NS], long long& n, long long e, const long long (&st)[NS]) {
  if (e == 1) return;
  if (n > 0) {
    bool merge = true;
    for (int k = 0; k < NS; ++k) merge = merge && str[k][n - 1] == e * st[k];
    if (merge) {
      ext[n - 1] *= e;
      for (int k = 0; k < NS; ++k) str[k][n - 1] = st[k];
      return;
    }
  }
  ext[n] = e;
  for (int k = 0; k < NS; ++k) str[k][n] = st[k];
  ++n;
}

// The kept and reduced axes of a reduction over storage images: in_str[a] is the input's element
// stride along axis a, out_str[a] the output's along kept axis a (ignored for reduced axes).
void fill_red_view(const std::vector<int64_t>& ext, int32_t rank, uint32_t mask, const long long* in_str,
                   const long long* out_str, unp::red_view_host& d) {
  long long* const kstrs[2] = {d.kstr, d.kost};
  long long* const rstrs[1] = {d.rstr};
  for (int32_t a = 0; a < rank; ++a) {
    if ((mask >> a) & 1u) {
      const long long st[1] = {in_str[a]};
      add_axis<1>(d.rext, rstrs, d.nr, ext[(size_t)a], st);
    } else {
      const long long st[2] = {in_str[a], out_str[a]};
      add_axis<2>(d.kext, kstrs, d.nk, ext[(size_t)a], st);
    }
  }
}

static_assert(sizeof(unp::red_view_host) == 44 * 8, "red_view_host mirrors the device's red_view");
static_assert(sizeof(unp::scan_view_host) == 29 * 8, "scan_view_host mirrors the device's scan_view");
static_assert(sizeof(unp::gather_view_host) == 35 * 8, "gather_view_host mirrors the device's gather_view");
static_assert(sizeof(unp::axes_desc_host) == 36 * 8, "axes_desc_host mirrors the device's axes_desc");

// At least n zeroed ticket counters.  Kernels leave every counter they use at zero, so a
// larger array is allocated afresh (and zeroed) only when a launch needs more strips.
int32_t ensure_counters(unp_exec* x, size_t n, unp_error* err) {
  if (n <= x->n_counters) return UNP_OK;
  if (x->counters) {
    hipFree(x->counters);
    x->counters = nullptr;
    x->n_counters = 0;
  }
  hipError_t e = hipMalloc((void**)&x->counters, n * sizeof(uint32_t));
  if (e != hipSuccess) return hip_fail(err, "hipMalloc(counters)", e);
  e = hipMemset(x->counters, 0, n * sizeof(uint32_t));
  if (e != hipSuccess) return hip_fail(err, "hipMemset(counters)", e);
  x->n_counters = n;
  return UNP_OK;
}

int32_t launch(unp_exec* x, size_t entry, uint32_t grid, void** params, hipStream_t s, unp_error* err) {
  const uint32_t threads = (uint32_t)(x->l.entries[entry].threads ? x->l.entries[entry].threads : x->l.threads);
  x->grid[0] = grid;
  x->grid[1] = x->grid[2] = 1;
  x->block[0] = threads;
  x->block[1] = x->block[2] = 1;
  x->last_entry = x->l.entries[entry].symbol;
  if (x->t_stop) {
    if ((uint64_t)grid * threads > 0xFFFFFFFFull) {
      set_error(err, UNP_INVALID_ARGUMENT, "a timed launch takes at most 2^32 - 1 work-items");
      return UNP_INVALID_ARGUMENT;
    }
    hipEvent_t start = x->t_first ? x->t_start : nullptr;
    x->t_first = false;
    const hipError_t e = hipExtModuleLaunchKernel(x->fns[entry], grid * threads, 1, 1, threads, 1, 1, 0, s, params,
                                                  nullptr, start, x->t_stop, 0);
    if (e != hipSuccess) return hip_fail(err, "hipExtModuleLaunchKernel", e);
    return UNP_OK;
  }
  const hipError_t e = hipModuleLaunchKernel(x->fns[entry], grid, 1, 1, threads, 1, 1, 0, s, params, nullptr);
  if (e != hipSuccess) return hip_fail(err, "hipModuleLaunchKernel", e);
  return UNP_OK;
}

// The pointer-launch entry for the arguments' alignment and row length (entries that read
// through storage-image strides are never picked here).
size_t pick(const unp_exec* x, bool fast_ok, bool wide = false) {
  const std::vector<unp::Entry>& es = x->l.entries;
  for (size_t i = 0; i < es.size(); ++i)
    if (!es[i].strided && es[i].fast == fast_ok && es[i].wide == wide) return i;
  for (size_t i = 0; i < es.size(); ++i)
    if (!es[i].strided && !es[i].fast && es[i].wide == wide) return i;
  size_t last = 0;
  for (size_t i = 0; i < es.size(); ++i)
    if (!es[i].strided) last = i;
  return last;
}

int64_t product(const std::vector<int64_t>& v, size_t from, size_t to) {
  int64_t p = 1;
  for (size_t i = from; i < to; ++i) p *= v[i];
  return p;
}

// A reduction with a pre-map body over NI inputs or a fused post: NI input buffers of the same
// shape, the output, then the extents.
int32_t run_xreduction(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  const unp_form& f = x->l.form;
  const size_t NI = (size_t)x->l.rx.n_inputs;
  Args A;
  int32_t rc = take_args(a, n, NI + 1, (size_t)f.rank, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, (size_t)f.rank, err);
  if (rc != UNP_OK) return rc;
  const uint32_t mask = x->l.axes_mask;
  long long outs = 1, count = 1;
  for (int32_t d = 0; d < f.rank; ++d) ((mask >> d) & 1u ? count : outs) *= A.ext[(size_t)d];
  if ((rc = need_buffers(A, outs > 0, err)) != UNP_OK) return rc;
  if (outs == 0) return UNP_OK;
  const int vec = 16 / (int)unp::kind_bytes(f.dtype);
  std::vector<uint64_t> ptrs(A.buf.begin(), A.buf.end());
  bool aligned = count % vec == 0;
  for (size_t k = 0; k < NI; ++k) aligned = aligned && aligned16(ptrs[k]);
  std::vector<void*> params;
  for (size_t k = 0; k <= NI; ++k) params.push_back(&ptrs[k]);
  const char sched = x->l.red_schedule;
  if (sched == 'r') {
    long long rows = outs, cols = count;
    params.push_back(&rows);
    params.push_back(&cols);
    const long long cap = (long long)x->cu_count * x->l.blocks_per_cu;
    return launch(x, aligned ? 0 : 1, (uint32_t)cap, params.data(), s, err);
  }
  if (sched == 'a') {
    const uint32_t grid = (uint32_t)(x->cu_count * x->l.blocks_per_cu);
    Ws w;
    uint32_t ep = 0;
    if ((rc = workspace(x, (size_t)grid * 16, true, 0, s, w, err)) != UNP_OK) return rc;
    if ((rc = next_epoch(x, s, ep, err)) != UNP_OK) return rc;
    long long nn = count;
    void* ws = w.ws;
    void* cnt = w.counter;
    waits_host wt = waits_of(x);
    params.push_back(&nn);
    params.push_back(&ws);
    params.push_back(&cnt);
    params.push_back(&ep);
    params.push_back(&wt);
    return launch(x, aligned ? 0 : 1, grid, params.data(), s, err);
  }
  unp::axes_desc_host d{};
  fill_axes_desc(A.ext, f.rank, mask, d);
  d.outs = outs;
  d.count = count;
  params.push_back(&d);
  const long long cap = (long long)x->cu_count * x->l.blocks_per_cu;
  return launch(x, 0, (uint32_t)cap, params.data(), s, err);
}

int32_t run_reduction(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  if (!x->l.rx.plain) return run_xreduction(x, a, n, s, err);
  const unp_form& f = x->l.form;
  const bool two = f.kind == UNP_FORM_ROW_REDUCE2;
  Args A;
  int32_t rc = take_args(a, n, two ? 3 : 2, (size_t)f.rank, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, (size_t)f.rank, err);
  if (rc != UNP_OK) return rc;
  const int vec = 16 / (int)unp::kind_bytes(f.dtype);
  const char sched = x->l.red_schedule;
  const uint32_t mask = x->l.axes_mask;
  if (sched == 'm' || sched == 'g' || sched == 'q') {
    // Output elements and reduced positions per output.
    long long outs = 1, count = 1;
    for (int32_t d = 0; d < f.rank; ++d) ((mask >> d) & 1u ? count : outs) *= A.ext[(size_t)d];
    if ((rc = need_buffers(A, outs > 0, err)) != UNP_OK) return rc;
    if (outs == 0) return UNP_OK;
    uint64_t in = A.buf[0], out = A.buf[1];
    if (sched == 'm') {
      // A x R x B: the kept axes before the reduced run, the run, the kept axes after it.
      int32_t fr = 0, lr = f.rank - 1;
      while (!((mask >> fr) & 1u)) ++fr;
      while (!((mask >> lr) & 1u)) --lr;
      long long a = product(A.ext, 0, (size_t)fr), r = product(A.ext, (size_t)fr, (size_t)lr + 1),
                b = product(A.ext, (size_t)lr + 1, (size_t)f.rank);
      const size_t entry = (b % vec == 0 && aligned16(in)) ? 0 : 1;
      const long long cw = 64LL * x->l.entries[entry].vec;
      const long long strips = a * ((b + cw - 1) / cw);
      // The grid is the device-class constant (cu_count * blocks_per_cu); the work is strips x S
      // items, S chunks of R: about one item per block, at least 16 rows per chunk, at most 1024
      // chunks.  Blocks stride over the items.
      const long long grid = (long long)x->cu_count * x->l.blocks_per_cu;
      long long S = (grid + strips - 1) / strips;
      S = std::min(S, std::max(1LL, r / 16));
      S = std::max(1LL, std::min(S, 1024LL));
      // A partial is one 8-byte tagged word per 4 bytes of accumulator.
      const size_t acc_bytes = (unp::kind_is_float(f.dtype) && (f.op0 == UNP_OP_SUM || f.op0 == UNP_OP_MEAN))
                                   ? 8
                                   : unp::kind_bytes(f.dtype);
      const size_t word_bytes = acc_bytes == 8 ? 16 : 8;
      void* ws = nullptr;
      void* cnt = nullptr;
      uint32_t ep = 0;
      if (S > 1) {
        Ws w;
        if ((rc = workspace(x, (size_t)(strips * S * cw) * word_bytes, false, (size_t)strips, s, w, err)) != UNP_OK)
          return rc;
        if ((rc = next_epoch(x, s, ep, err)) != UNP_OK) return rc;
        ws = w.ws;
        cnt = w.counters;
      }
      waits_host wt = waits_of(x);
      void* params[] = {&in, &out, &a, &r, &b, &S, &ws, &cnt, &ep, &wt};
      return launch(x, entry, (uint32_t)grid, params, s, err);
    }
    const long long cap = (long long)x->cu_count * x->l.blocks_per_cu;
    if (sched == 'q') {
      // The serial product (a lane per output) takes the storage-image descriptor, here with the
      // row-major strides of the input and of the kept-axes output.
      std::vector<long long> in_str((size_t)f.rank), out_str((size_t)f.rank, 0);
      long long si = 1, so = 1;
      for (int32_t k = f.rank - 1; k >= 0; --k) {
        in_str[(size_t)k] = si;
        si *= A.ext[(size_t)k];
        if (!((mask >> k) & 1u)) {
          out_str[(size_t)k] = so;
          so *= A.ext[(size_t)k];
        }
      }
      unp::red_view_host d{};
      fill_red_view(A.ext, f.rank, mask, in_str.data(), out_str.data(), d);
      d.outs = outs;
      d.count = count;
      void* params[] = {&in, &out, &d};
      return launch(x, 0, (uint32_t)cap, params, s, err);
    }
    // Any other mask: a wave per output.
    unp::axes_desc_host d{};
    fill_axes_desc(A.ext, f.rank, mask, d);
    d.outs = outs;
    d.count = count;
    void* params[] = {&in, &out, &d};
    return launch(x, 0, (uint32_t)cap, params, s, err);
  }
  const long long rows = product(A.ext, 0, (size_t)f.reduced_from);
  const long long cols = product(A.ext, (size_t)f.reduced_from, (size_t)f.rank);
  if ((rc = need_buffers(A, rows > 0, err)) != UNP_OK) return rc;
  if (rows == 0) return UNP_OK;
  uint64_t in = A.buf[0], o0 = A.buf[1], o1 = two ? A.buf[2] : A.buf[1];
  const size_t entry = pick(x, cols % vec == 0 && aligned16(in), !x->l.reduce_all && cols > unp::kWideRow);
  const uint32_t grid = (uint32_t)(x->cu_count * x->l.blocks_per_cu);
  if (x->l.reduce_all) {
    // Up to two 8-byte tagged words per block partial.
    Ws w;
    uint32_t ep = 0;
    if ((rc = workspace(x, (size_t)grid * 16, true, 0, s, w, err)) != UNP_OK) return rc;
    if ((rc = next_epoch(x, s, ep, err)) != UNP_OK) return rc;
    long long nn = cols;
    void* ws = w.ws;
    void* cnt = w.counter;
    waits_host wt = waits_of(x);
    void* params[] = {&in, &o0, &nn, &ws, &cnt, &ep, &wt};
    return launch(x, entry, grid, params, s, err);
  }
  long long r = rows, c = cols;
  void* params[] = {&in, &o0, &o1, &r, &c};
  return launch(x, entry, grid, params, s, err);
}

// A scan with a pre-map body and a fused post: n inputs of one shape, then the output.
int32_t run_xscan(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  const unp_form& f = x->l.form;
  const size_t NI = (size_t)x->l.rx.n_inputs;
  Args A;
  int32_t rc = take_args(a, n, NI + 1, (size_t)f.rank, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, (size_t)f.rank, err);
  if (rc != UNP_OK) return rc;
  std::vector<uint64_t> ptrs(A.buf.begin(), A.buf.end());
  std::vector<void*> params;
  for (size_t k = 0; k <= NI; ++k) params.push_back(&ptrs[k]);
  const uint32_t grid = (uint32_t)(x->cu_count * x->l.blocks_per_cu);
  if (x->l.serial_scan) {
    const size_t ax = (size_t)x->l.scan_axis;
    long long a0 = product(A.ext, 0, ax), S = A.ext[ax], b0 = product(A.ext, ax + 1, (size_t)f.rank);
    if ((rc = need_buffers(A, a0 > 0 && S > 0 && b0 > 0, err)) != UNP_OK) return rc;
    if (a0 == 0 || S == 0 || b0 == 0) return UNP_OK;
    params.push_back(&a0);
    params.push_back(&S);
    params.push_back(&b0);
    return launch(x, 0, grid, params.data(), s, err);
  }
  long long rows = product(A.ext, 0, (size_t)f.rank - 1);
  long long cols = A.ext[(size_t)f.rank - 1];
  if ((rc = need_buffers(A, rows > 0 && cols > 0, err)) != UNP_OK) return rc;
  if (rows == 0 || cols == 0) return UNP_OK;
  const unp::Entry& en = x->l.entries[0];
  const long long tile = 64LL * en.k * en.wpb;
  const unsigned long long tiles = (unsigned long long)rows * (unsigned long long)((cols + tile - 1) / tile);
  if (tiles + grid >= (1ull << 31)) {
    set_error(err, UNP_INVALID_ARGUMENT, "too many scan tiles for one launch");
    return UNP_INVALID_ARGUMENT;
  }
  Ws w;
  if ((rc = workspace(x, (size_t)tiles * unp::kScanStatusWords * 8, true, 0, s, w, err)) != UNP_OK) return rc;
  waits_host wt = waits_of(x);
  uint32_t ep = 0;
  if ((rc = next_epoch(x, s, ep, err)) != UNP_OK) return rc;
  uint32_t tb = x->fixed ? 0 : x->ticket_base;
  void* st = w.ws;
  void* cnt = w.counter;
  params.push_back(&rows);
  params.push_back(&cols);
  params.push_back(&st);
  params.push_back(&cnt);
  params.push_back(&tb);
  params.push_back(&ep);
  params.push_back(&wt);
  rc = launch(x, 0, grid, params.data(), s, err);
  // One ticket per tile, plus the one failing draw that ends each block.
  if (rc == UNP_OK && !x->fixed) x->ticket_base = (uint32_t)(x->ticket_base + (uint32_t)(tiles + grid));
  return rc;
}

int32_t run_scan(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  if (!x->l.rx.plain) return run_xscan(x, a, n, s, err);
  const unp_form& f = x->l.form;
  Args A;
  int32_t rc = take_args(a, n, 2, (size_t)f.rank, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, (size_t)f.rank, err);
  if (rc != UNP_OK) return rc;
  if (x->l.serial_scan) {
    // The input as A x S x B around the scanned axis; one lane per column.
    const size_t ax = (size_t)x->l.scan_axis;
    long long a0 = product(A.ext, 0, ax), S = A.ext[ax], b0 = product(A.ext, ax + 1, (size_t)f.rank);
    if ((rc = need_buffers(A, a0 > 0 && S > 0 && b0 > 0, err)) != UNP_OK) return rc;
    if (a0 == 0 || S == 0 || b0 == 0) return UNP_OK;
    uint64_t in = A.buf[0], out = A.buf[1];
    void* params[] = {&in, &out, &a0, &S, &b0};
    return launch(x, 0, (uint32_t)(x->cu_count * x->l.blocks_per_cu), params, s, err);
  }
  long long rows = product(A.ext, 0, (size_t)f.rank - 1);
  long long cols = A.ext[(size_t)f.rank - 1];
  if ((rc = need_buffers(A, rows > 0 && cols > 0, err)) != UNP_OK) return rc;
  if (rows == 0 || cols == 0) return UNP_OK;
  const int vec = 16 / (int)unp::kind_bytes(f.dtype);
  uint64_t in = A.buf[0], out = A.buf[1];
  const size_t entry = pick(x, cols % vec == 0 && aligned16(in) && aligned16(out));
  const unp::Entry& en = x->l.entries[entry];
  // A block tile: wpb (consumer) waves x 64 lanes x vec x k positions of one row.
  const long long tile = 64LL * en.vec * en.k * en.wpb;
  const unsigned long long tiles = (unsigned long long)rows * (unsigned long long)((cols + tile - 1) / tile);
  const uint32_t grid = (uint32_t)(x->cu_count * (en.blocks_per_cu ? en.blocks_per_cu : x->l.blocks_per_cu));
  if (tiles + grid >= (1ull << 31)) {
    set_error(err, UNP_INVALID_ARGUMENT, "too many scan tiles for one launch");
    return UNP_INVALID_ARGUMENT;
  }
  Ws w;
  if ((rc = workspace(x, (size_t)tiles * unp::kScanStatusWords * 8, true, 0, s, w, err)) != UNP_OK) return rc;
  waits_host wt = waits_of(x);
  uint32_t ep = 0;
  if ((rc = next_epoch(x, s, ep, err)) != UNP_OK) return rc;
  if (x->fixed) {
    // The scratch was just cleared: epoch 1 and tickets from 0, and no state kept for the next call.
    uint32_t tb = 0;
    void* st = w.ws;
    void* cnt = w.counter;
    void* params[] = {&in, &out, &rows, &cols, &st, &cnt, &tb, &ep, &wt};
    return launch(x, entry, grid, params, s, err);
  }
  uint32_t tb = x->ticket_base;
  void* st = w.ws;
  void* cnt = w.counter;
  void* params[] = {&in, &out, &rows, &cols, &st, &cnt, &tb, &ep, &wt};
  rc = launch(x, entry, grid, params, s, err);
  // One ticket per tile, plus the one failing draw that ends each block.
  if (rc == UNP_OK) x->ticket_base = (uint32_t)(x->ticket_base + (uint32_t)(tiles + grid));
  return rc;
}

int32_t run_row_reduce(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  const unp::RowReduceSpec& sp = x->l.rr;
  const size_t ni = (size_t)sp.n_inputs, r = (size_t)sp.rank;
  Args A;
  int32_t rc = take_args(a, n, ni + 1, r, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, r, err);
  if (rc != UNP_OK) return rc;
  long long rows = product(A.ext, 0, r - 1);
  long long cols = A.ext[r - 1];
  if ((rc = need_buffers(A, rows > 0 && cols > 0, err)) != UNP_OK) return rc;
  if (rows == 0 || cols == 0) return UNP_OK;
  const int vec = 16 / (int)unp::kind_bytes(sp.dtype);
  bool aligned = cols % vec == 0;
  for (uint64_t p : A.buf) aligned = aligned && aligned16(p);
  // entries: 0 the row in registers (4 vectors per thread), 1 in registers (8 vectors per
  // thread), 2 vector passes, 3 scalar passes
  const size_t entry = !aligned ? 3 : (cols <= 256LL * vec * 4 ? 0 : (cols <= 256LL * vec * 8 ? 1 : 2));
  // As many blocks as the CUs hold at once (at most blocks_per_cu each), so no blocks start late
  // as a tail that runs at a fraction of the occupancy.
  const int held = x->resident[entry];
  const long long cap = (long long)x->cu_count * (held > 0 && held < x->l.blocks_per_cu ? held : x->l.blocks_per_cu);
  const uint32_t grid = (uint32_t)cap;
  std::vector<void*> params;
  std::vector<uint64_t> ptrs(A.buf.begin(), A.buf.end());
  for (size_t i = 0; i < ptrs.size(); ++i) params.push_back(&ptrs[i]);
  params.push_back(&rows);
  params.push_back(&cols);
  return launch(x, entry, grid, params.data(), s, err);
}

// The general gather's launch: the descriptor from each input's strides (istr[k][d] over the output
// coordinates), the output's, and the source extent.
int32_t launch_gather_x(unp_exec* x, const std::vector<uint64_t>& ptrs, const unp::gather_x_view_host& v,
                        int64_t raw_src, hipStream_t s, unp_error* err) {
  const unp_form& f = x->l.form;
  if (v.outs == 0) return UNP_OK;
  int64_t src = raw_src;
  if (f.index_dtype == UNP_I32) src = (int64_t)(int32_t)(uint32_t)(uint64_t)raw_src;
  else if (f.index_dtype == UNP_U32) src = (int64_t)(uint32_t)(uint64_t)raw_src;
  if (src <= 0 && f.oob == UNP_OOB_CLAMP) {
    set_error(err, UNP_INVALID_ARGUMENT, "a Clamp gather needs a source extent of at least 1");
    return UNP_INVALID_ARGUMENT;
  }
  int32_t e32 = (int32_t)src;
  uint32_t eu32 = (uint32_t)src;
  long long e64 = src;
  std::vector<uint64_t> p(ptrs);
  std::vector<void*> params;
  for (auto& q : p) params.push_back(&q);
  unp::gather_x_view_host vv = v;
  params.push_back(&vv);
  params.push_back(f.index_dtype == UNP_I32 ? (void*)&e32 : (f.index_dtype == UNP_U32 ? (void*)&eu32 : (void*)&e64));
  return launch(x, 0, (uint32_t)(x->cu_count * x->l.blocks_per_cu), params.data(), s, err);
}

// A general gather from device addresses: every input dense over the output's shape, the
// gathered one with src_extent along the axis, the index 1-D along the axis (broadcast over the
// others, as the row gather reads it).
int32_t run_gather_x(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  const unp_form& f = x->l.form;
  const size_t NI = (size_t)x->l.gx.n_inputs;
  Args A;
  int32_t rc = take_args(a, n, NI + 1, (size_t)f.rank + 1, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, (size_t)f.rank, err);
  if (rc != UNP_OK) return rc;
  const int ax = x->l.scan_axis, ix = x->l.gx.index_slot, data = f.data_slot;
  unp::gather_x_view_host v{};
  v.rank = f.rank;
  v.axis = ax;
  v.outs = 1;
  for (int d = 0; d < f.rank; ++d) {
    v.ext[d] = A.ext[(size_t)d];
    v.outs *= v.ext[d];
  }
  if ((rc = need_buffers(A, v.outs > 0, err)) != UNP_OK) return rc;
  int64_t src = (int64_t)A.ext[(size_t)f.rank];
  if (f.index_dtype == UNP_I32) src = (int64_t)(int32_t)(uint32_t)(uint64_t)src;
  else if (f.index_dtype == UNP_U32) src = (int64_t)(uint32_t)(uint64_t)src;
  for (size_t k = 0; k <= NI; ++k) {
    long long st = 1;
    for (int d = f.rank - 1; d >= 0; --d) {
      long long e = v.ext[d];
      if ((int)k == data && d == ax) e = src > 0 ? src : 0;
      if (k == NI) v.ostr[d] = st;
      else if ((int)k == ix) v.istr[k][d] = d == ax ? 1 : 0;
      else v.istr[k][d] = st;
      st *= e;
    }
  }
  std::vector<uint64_t> ptrs(A.buf.begin(), A.buf.end());
  return launch_gather_x(x, ptrs, v, (int64_t)A.ext[(size_t)f.rank], s, err);
}

int32_t run_gather(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  if (!x->l.gx.plain) return run_gather_x(x, a, n, s, err);
  const unp_form& f = x->l.form;
  Args A;
  int32_t rc = take_args(a, n, 3, (size_t)f.rank + 1, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, (size_t)f.rank, err);
  if (rc != UNP_OK) return rc;
  // The output as A x NI rows around the gathered axis (A = 1 for axis 0).
  const size_t ax = (size_t)x->l.scan_axis;
  const long long ni = A.ext[ax];
  const long long n_rows = product(A.ext, 0, ax + 1);
  const long long row_elems = product(A.ext, ax + 1, (size_t)f.rank);
  const long long row_bytes = row_elems * (long long)unp::kind_bytes(f.dtype);
  if ((rc = need_buffers(A, n_rows > 0 && row_bytes > 0, err)) != UNP_OK) return rc;
  if (n_rows == 0 || row_bytes == 0) return UNP_OK;
  uint64_t table = A.buf[f.data_slot == 0 ? 0 : 1];
  uint64_t ids = A.buf[f.data_slot == 0 ? 1 : 0];
  uint64_t out = A.buf[2];
  const uint64_t raw_ext = (uint64_t)A.ext[(size_t)f.rank];
  int32_t ext32 = 0;
  uint32_t extu32 = 0;
  long long ext64 = 0;
  bool empty_source = false;
  if (f.index_dtype == UNP_I32) {
    ext32 = (int32_t)(uint32_t)raw_ext;
    empty_source = ext32 <= 0;
  } else if (f.index_dtype == UNP_U32) {
    extu32 = (uint32_t)raw_ext;
    empty_source = extu32 == 0;
  } else {
    ext64 = (long long)raw_ext;
    empty_source = ext64 <= 0;
  }
  if (empty_source && f.oob == UNP_OOB_CLAMP) {
    // Clamping into an empty source has no row to read.
    set_error(err, UNP_INVALID_ARGUMENT, "a Clamp gather needs a source extent of at least 1");
    return UNP_INVALID_ARGUMENT;
  }
  const size_t entry = pick(x, row_bytes % 16 == 0 && aligned16(table) && aligned16(out));
  const int bpc = x->l.entries[entry].blocks_per_cu ? x->l.entries[entry].blocks_per_cu : x->l.blocks_per_cu;
  const uint32_t grid = (uint32_t)(x->cu_count * bpc);
  long long nr = n_rows, rb = row_bytes, nib = ni;
  void* ext_arg = f.index_dtype == UNP_I32 ? (void*)&ext32 : (f.index_dtype == UNP_U32 ? (void*)&extu32 : (void*)&ext64);
  void* params[] = {&table, &ids, &out, &nr, &rb, ext_arg, &nib};
  return launch(x, entry, grid, params, s, err);
}

// The elementwise op's strided launch: the descriptor holds the output's extents and strides and
// every input's strides over the output's axes.
int32_t launch_elementwise_strided(unp_exec* x, const std::vector<uint64_t>& ptrs, const unp::gather_x_view_host& v,
                                   hipStream_t s, unp_error* err) {
  if (v.outs == 0) return UNP_OK;
  std::vector<uint64_t> p(ptrs);
  std::vector<void*> params;
  for (auto& q : p) params.push_back(&q);
  unp::gather_x_view_host vv = v;
  params.push_back(&vv);
  const long long blocks = (v.outs + 255) / 256;
  const uint32_t grid = (uint32_t)std::min<long long>(blocks, (long long)x->cu_count * x->l.blocks_per_cu);
  size_t entry = 0;
  while (entry + 1 < x->l.entries.size() && !x->l.entries[entry].strided) ++entry;
  return launch(x, entry, grid, params.data(), s, err);
}

// An elementwise op from device addresses: every buffer dense row-major in its own shape, a
// permuted input in its own axis order (the shape whose axis perm[d] has the output's extent d).
int32_t run_elementwise(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  const unp_form& f = x->l.form;
  const unp::ElementwiseExpr& ew = x->l.ew;
  const size_t NI = (size_t)ew.n_inputs;
  Args A;
  int32_t rc = take_args(a, n, NI + 1, (size_t)f.rank, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, (size_t)f.rank, err);
  if (rc != UNP_OK) return rc;
  const long long total = product(A.ext, 0, (size_t)f.rank);
  if ((rc = need_buffers(A, total > 0, err)) != UNP_OK) return rc;
  if (total == 0) return UNP_OK;
  std::vector<uint64_t> ptrs(A.buf.begin(), A.buf.end());
  if (!ew.permuted()) {
    bool al = true;
    for (uint64_t q : ptrs) al = al && aligned16(q);
    const size_t entry = pick(x, al);
    const long long vec = x->l.entries[entry].vec, np = total / vec;
    const long long lanes = std::max(np, total - np * vec);
    const uint32_t grid =
        (uint32_t)std::max<long long>(1, std::min<long long>((lanes + 255) / 256, (long long)x->cu_count * x->l.blocks_per_cu));
    std::vector<void*> params;
    for (auto& q : ptrs) params.push_back(&q);
    long long nn = total;
    params.push_back(&nn);
    return launch(x, entry, grid, params.data(), s, err);
  }
  unp::gather_x_view_host v{};
  v.rank = f.rank;
  v.outs = total;
  long long st = 1;
  for (int d = f.rank - 1; d >= 0; --d) {
    v.ext[d] = A.ext[(size_t)d];
    v.ostr[d] = st;
    st *= v.ext[d];
  }
  for (size_t k = 0; k < NI; ++k) {
    // Input k's own shape and row-major strides, then the stride of iteration axis d is that of
    // its axis perm[d].
    long long shape[8], pstr[8];
    for (int d = 0; d < f.rank; ++d) shape[ew.perms.empty() ? d : ew.perms[k][(size_t)d]] = v.ext[d];
    long long ps = 1;
    for (int a2 = f.rank - 1; a2 >= 0; --a2) {
      pstr[a2] = ps;
      ps *= shape[a2];
    }
    for (int d = 0; d < f.rank; ++d) v.istr[k][d] = pstr[ew.perms.empty() ? d : ew.perms[k][(size_t)d]];
  }
  return launch_elementwise_strided(x, ptrs, v, s, err);
}

int32_t run_dequant(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  Args A;
  int32_t rc = take_args(a, n, 4, 2, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, 2, err);
  if (rc != UNP_OK) return rc;
  long long rows = A.ext[0], cols = A.ext[1];
  if ((rc = need_buffers(A, rows > 0 && cols > 0, err)) != UNP_OK) return rc;
  if (rows == 0 || cols == 0) return UNP_OK;
  uint64_t q = A.buf[0], sc = A.buf[1], zp = A.buf[2], out = A.buf[3];
  const long long group = x->l.form.group;
  const bool fast_ok = cols % group == 0 && (q & 3) == 0 && aligned16(out) && (sc & 1) == 0;
  size_t entry = pick(x, fast_ok);
  if (x->l.entries[entry].fast && !fast_ok) entry = x->l.entries.size() - 1;
  const uint32_t grid = (uint32_t)(x->cu_count * x->l.blocks_per_cu);
  void* params[] = {&q, &sc, &zp, &out, &rows, &cols};
  return launch(x, entry, grid, params, s, err);
}

// The dequantizing GEMM: w, zero, scale, x, out, then R, K, C.  The MFMA entry takes whole
// groups, 4-column rows of x and aligned operands; anything else runs the serial entry.
bool ends_with(const std::string& s, const char* tail) {
  const size_t n = std::strlen(tail);
  return s.size() > n && s.compare(s.size() - n, n, tail) == 0;
}

// The two-launch dequant-GEMM schedules: the prep entry repacks x into the workspace (Cp columns,
// its grid covering groups x (Cp / cols_per_prep_block)) and zeroes out when K is split; then the
// main entry runs over `blocks` blocks with S splits of K.
int32_t run_repacked(unp_exec* x, size_t prep, size_t main, uint64_t w, uint64_t zp, uint64_t sc, uint64_t xa,
                     uint64_t out, long long R, long long K, long long C, long long Cp, long long prep_cols,
                     long long S, long long blocks, hipStream_t s, unp_error* err) {
  const long long group = x->l.form.group, ng = K / group, xbytes = x->l.form.dtype == UNP_I32 ? 4 : 1;
  if (blocks > 0x7FFFFFFFLL || ng * (Cp / prep_cols) > 0x7FFFFFFFLL) {
    set_error(err, UNP_INVALID_ARGUMENT, "dequant GEMM shape too large for one launch");
    return UNP_INVALID_ARGUMENT;
  }
  // x' (K x Cp x digit planes bytes), then the group column sums (ng x Cp u32, 64 spare).
  const size_t xp_bytes = (size_t)K * (size_t)Cp * (size_t)xbytes;
  Ws wsp;
  int32_t rc = workspace(x, xp_bytes + ((size_t)ng * (size_t)Cp + 64) * 4, false, 0, s, wsp, err);
  if (rc != UNP_OK) return rc;
  uint64_t xp = (uint64_t)wsp.ws, xs = xp + xp_bytes;
  long long Kp = K, Cc = C, Cpp = Cp, G = group, n_out = S > 1 ? R * C : 0;
  void* pparams[] = {&xa, &xp, &xs, &Kp, &Cc, &Cpp, &G, &out, &n_out};
  // Device-class grids: the prep's blocks stride over its (group, column slab) items and the main
  // kernel's over its `blocks` items, as many blocks as the entry keeps resident per CU.
  if ((rc = launch(x, prep, (uint32_t)(x->cu_count * x->l.blocks_per_cu), pparams, s, err)) != UNP_OK) return rc;
  // The streaming entry keeps one block per item: an item loop around its LDS pipeline made it spill.
  const bool per_item = ends_with(x->l.entries[main].symbol, "_stream");
  const int bpc = x->l.entries[main].blocks_per_cu ? x->l.entries[main].blocks_per_cu : 2;
  void* mparams[] = {&w, &zp, &sc, &xp, &xs, &out, &R, &K, &C, &Cpp, &S};
  return launch(x, main, (uint32_t)(per_item ? blocks : x->cu_count * bpc), mparams, s, err);
}

int32_t run_dequant_gemm(unp_exec* x, const unp_arg* a, size_t n, hipStream_t s, unp_error* err) {
  Args A;
  int32_t rc = take_args(a, n, 5, 3, A, err);
  if (rc == UNP_OK) rc = extents_i32(A, 3, err);
  if (rc != UNP_OK) return rc;
  long long R = A.ext[0], K = A.ext[1], C = A.ext[2];
  if ((rc = need_buffers(A, R > 0 && C > 0, err)) != UNP_OK) return rc;
  if (R == 0 || C == 0) return UNP_OK;
  uint64_t w = A.buf[0], zp = A.buf[1], sc = A.buf[2], xa = A.buf[3], out = A.buf[4];
  const long long group = x->l.form.group;
  const bool x32 = x->l.form.dtype == UNP_I32;
  const long long xbytes = x32 ? 4 : 1;
  size_t stream = SIZE_MAX, prep = SIZE_MAX, dec = SIZE_MAX, prep16 = SIZE_MAX, mfma = SIZE_MAX, any = SIZE_MAX;
  for (size_t i = 0; i < x->l.entries.size(); ++i) {
    const std::string& sym = x->l.entries[i].symbol;
    if (ends_with(sym, "_stream")) stream = i;
    if (ends_with(sym, "_prep")) prep = i;
    if (ends_with(sym, "_prep16")) prep16 = i;
    if (ends_with(sym, "_mfma")) mfma = i;
    if (ends_with(sym, "_any")) any = i;
    // The decode entry whose column tiles first cover C, else the widest (entries ascend).
    const int cols = x->l.entries[i].cols;
    if (cols > 0 && (dec == SIZE_MAX || x->l.entries[dec].cols < C)) dec = i;
  }
  // The two-launch schedules need whole groups, a 16-byte aligned w and aligned operands.
  const bool whole = K > 0 && K % group == 0 && (w & 15) == 0 && (zp & 3) == 0 && (sc & 3) == 0 &&
                     (out & 3) == 0 && (xa & (x32 ? 3 : 0)) == 0;
  // Decode up to 64 columns for I8 activations (the streaming entry's 128 x 128 tiles win beyond),
  // up to 128 for I32; its buffer loads take 32-bit offsets.
  if (dec != SIZE_MAX && prep16 != SIZE_MAX && whole && C <= (x32 ? 128 : 64)) {
    const long long bm = x->l.entries[dec].vec, bn = x->l.entries[dec].cols, maxg = x->l.entries[dec].k;
    const long long ng = K / group, Cp = (C + bn - 1) / bn * bn;  // whole column tiles of the entry
    if (R * (K / 2) < 0x7FFFFFFFLL && K * Cp * xbytes < 0x7FFFFFFFLL) {
      const long long tiles_r = (R + bm - 1) / bm, tiles_c = Cp / bn;
      // Splits of K: about the entry's blocks per CU (two by default), at most maxg groups per
      // split, at least one.
      const long long bpc = x->l.entries[dec].blocks_per_cu ? x->l.entries[dec].blocks_per_cu : 2;
      long long S = (bpc * x->cu_count + tiles_r * tiles_c - 1) / (tiles_r * tiles_c);
      S = std::max(S, (ng + maxg - 1) / maxg);
      S = std::max(1LL, std::min(S, ng));
      const long long blocks = (tiles_r + 7) / 8 * 8 * S * tiles_c;
      return run_repacked(x, prep16, dec, w, zp, sc, xa, out, R, K, C, Cp, 16, S, blocks, s, err);
    }
  }
  if (stream != SIZE_MAX && prep != SIZE_MAX && whole) {
    // Streaming: the LDS-staged MFMA kernel over (row tile, split) x column tiles.
    const long long bm = x->l.entries[stream].vec, bn = x->l.entries[stream].k;
    // Whole column tiles of the entry and whole 64-column prep slabs (bn is 32, 64 or 128).
    const long long cw = std::max(bn, 64LL), ng = K / group, Cp = (C + cw - 1) / cw * cw;
    // Its zero-point pass reads scales, zero points and column sums by 32-bit byte offsets,
    // up to a row tile and a 32-group step past their ends.
    if ((R + 256) * ng * 4 < 0x7FFFFFFFLL && (ng + 32) * Cp * 4 < 0x7FFFFFFFLL) {
      const long long tiles_r = (R + bm - 1) / bm, tiles_c = (C + bn - 1) / bn;
      // Splits of K: enough blocks for two per CU, at least four groups per split.
      long long S = (2LL * x->cu_count + tiles_r * tiles_c - 1) / (tiles_r * tiles_c);
      S = std::max(1LL, std::min(S, ng / 4));
      const long long blocks = (tiles_r * S + 7) / 8 * 8 * tiles_c;
      return run_repacked(x, prep, stream, w, zp, sc, xa, out, R, K, C, Cp, 64, S, blocks, s, err);
    }
  }
  // One launch: the LDS-transpose MFMA entry when its operands line up, else the serial entry.
  const long long tiles = ((R + 63) / 64) * ((C + 63) / 64);
  const bool mfma_ok = mfma != SIZE_MAX && K % group == 0 && C % 4 == 0 && xa % (x32 ? 16 : 4) == 0 &&
                       (w & 7) == 0 && (zp & 3) == 0 && (sc & 3) == 0 && (out & 3) == 0 && tiles <= 0x7FFFFFFFLL;
  const size_t entry = mfma_ok ? mfma : any;
  // Both take a device-class grid; the MFMA entry's blocks stride over its 64 x 64 tiles.
  const uint32_t grid = (uint32_t)(x->cu_count * (mfma_ok ? 4 : x->l.blocks_per_cu));
  void* params[] = {&w, &zp, &sc, &xa, &out, &R, &K, &C};
  return launch(x, entry, grid, params, s, err);
}

}  // namespace

// Element bits of buffer parameter b of a form: the element kinds of its storage images.
static int view_elem_bits(const unp::Lowered& l, size_t b) {
  const unp_form& f = l.form;
  int32_t k = f.dtype;
  if (f.kind == UNP_FORM_GATHER) {
    // buffer b of a gather: the index slot carries the index kind, every other buffer the data's
    // (the plain gather's index is the input that is not data_slot)
    const bool index = l.gx.plain ? ((b == 0 || b == 1) && (int)b != f.data_slot) : (int)b == l.gx.index_slot;
    k = index ? f.index_dtype : f.dtype;
  } else if (f.kind == UNP_FORM_DEQUANT4) {
    const int32_t ks[4] = {f.q_kind, UNP_F16, f.z_kind, f.out_kind};
    if (b < 4) k = ks[b];
  } else if (f.kind == UNP_FORM_DEQUANT_GEMM) {
    const int32_t ks[5] = {f.q_kind, UNP_I32, UNP_I32, f.dtype, UNP_I32};
    if (b < 5) k = ks[b];
  }
  const size_t by = unp::kind_bytes(k);
  return by ? (int)(8 * by) : 4;  // the sub-byte kinds this backend reads are 4-bit
}

namespace {

int64_t low_i32(int64_t v) { return (int64_t)(int32_t)(uint32_t)(uint64_t)v; }

// The buffer and scalar parameters of a lowered form's KernelFn.
void param_counts(const unp_exec* x, size_t& nbuf, size_t& nscal) {
  const unp_form& f = x->l.form;
  nbuf = nscal = 0;
  switch (f.kind) {
    case UNP_FORM_REDUCTION: nbuf = (size_t)x->l.rx.n_inputs + 1; nscal = (size_t)f.rank; break;
    case UNP_FORM_ROW_REDUCE2: nbuf = 3; nscal = 2; break;
    case UNP_FORM_SCAN: nbuf = (size_t)x->l.rx.n_inputs + 1; nscal = (size_t)f.rank; break;
    case UNP_FORM_GATHER: nbuf = (size_t)x->l.gx.n_inputs + 1; nscal = (size_t)f.rank + 1; break;
    case UNP_FORM_ROW_REDUCE: nbuf = (size_t)x->l.rr.n_inputs + 1; nscal = (size_t)x->l.rr.rank; break;
    case UNP_FORM_DEQUANT4: nbuf = 4; nscal = 2; break;
    case UNP_FORM_DEQUANT_GEMM: nbuf = 5; nscal = 3; break;
    case UNP_FORM_ELEMENTWISE: nbuf = (size_t)x->l.ew.n_inputs + 1; nscal = (size_t)f.rank; break;
    default: break;
  }
}

// The shape a buffer parameter's view must have, from the form and the extent scalars (the
// extents every access of the KernelFn ranges over).  A reduction's output may also take the
// keepdim shape (the input's rank, its reduced axes of extent 1); a gather's table has the
// output's extents except along the gathered axis, where it holds at least src_extent rows.
struct Want {
  std::vector<int64_t> shape;
  std::vector<int64_t> keepdim;  // empty: no alternative
  int table_axis = -1;
  int64_t table_rows = 0;
};

int64_t ceil_div(int64_t a, int64_t b) { return b > 0 ? (a + b - 1) / b : 0; }

// The gather's source extent as its index type reads it (negative: no row is ever read).
int64_t gather_src_extent(const unp_form& f, int64_t raw) {
  if (f.index_dtype == UNP_I32) return low_i32(raw);
  if (f.index_dtype == UNP_U32) return (int64_t)(uint32_t)(uint64_t)raw;
  return raw;
}

std::vector<Want> wanted_shapes(const unp_exec* x, const std::vector<int64_t>& ext, const int64_t* sc) {
  const unp_form& f = x->l.form;
  std::vector<Want> w;
  auto one = [&](std::vector<int64_t> s) {
    Want a;
    a.shape = std::move(s);
    w.push_back(a);
  };
  switch (f.kind) {
    case UNP_FORM_REDUCTION:
    case UNP_FORM_ROW_REDUCE2: {
      const bool two = f.kind == UNP_FORM_ROW_REDUCE2;
      const size_t nin = two ? 1 : (size_t)x->l.rx.n_inputs;
      for (size_t k = 0; k < nin; ++k) one(ext);
      Want o;
      std::vector<int64_t> kd(ext);
      for (int32_t d = 0; d < f.rank; ++d) {
        if ((x->l.axes_mask >> d) & 1u) kd[(size_t)d] = 1;
        else o.shape.push_back(ext[(size_t)d]);
      }
      if (!two) o.keepdim = kd;
      w.push_back(o);
      if (two) w.push_back(o);
      break;
    }
    case UNP_FORM_SCAN:
      for (int32_t k = 0; k <= x->l.rx.n_inputs; ++k) one(ext);  // the inputs and the output
      break;
    case UNP_FORM_GATHER: {
      // The gathered input (data_slot) is the table; every other input, the index among them,
      // has the output's shape.
      Want t;
      t.shape = ext;
      t.table_axis = x->l.scan_axis;
      t.table_rows = std::max<int64_t>(0, gather_src_extent(f, sc[f.rank]));
      for (int32_t k = 0; k < x->l.gx.n_inputs; ++k) {
        if (k == f.data_slot) w.push_back(t);
        else one(ext);
      }
      one(ext);
      break;
    }
    case UNP_FORM_ROW_REDUCE:
      for (int32_t k = 0; k <= x->l.rr.n_inputs; ++k) one(ext);
      break;
    case UNP_FORM_DEQUANT4: {
      const int64_t R = ext[0], C = ext[1], ng = ceil_div(C, f.group);
      one({R * C});
      one({R * ng});
      one({R * ng});
      one({R * C});
      break;
    }
    case UNP_FORM_ELEMENTWISE: {
      // Input k in its own axis order: its axis perm[d] has the output's extent d.
      for (int32_t k = 0; k < x->l.ew.n_inputs; ++k) {
        std::vector<int64_t> s(ext);
        if (!x->l.ew.perms.empty())
          for (int32_t d = 0; d < f.rank; ++d) s[(size_t)x->l.ew.perms[(size_t)k][(size_t)d]] = ext[(size_t)d];
        one(s);
      }
      one(ext);
      break;
    }
    case UNP_FORM_DEQUANT_GEMM: {
      const int64_t R = ext[0], K = ext[1], C = ext[2], ng = ceil_div(K, f.group);
      one({R * K});
      one({R * ng});
      one({R * ng});
      one({K * C});
      one({R * C});
      break;
    }
    default:
      break;
  }
  return w;
}

std::string shape_text(const int64_t* s, size_t n) {
  std::string t = "[";
  for (size_t d = 0; d < n; ++d) t += (d ? ", " : "") + std::to_string(s[d]);
  return t + "]";
}

bool shape_is(const unp_view& v, const std::vector<int64_t>& s) {
  if ((size_t)v.rank != s.size()) return false;
  for (size_t d = 0; d < s.size(); ++d)
    if (v.shape[d] != s[d]) return false;
  return true;
}

// Whether view v has the shape `want` asks for; `why` says how it differs.
bool shape_ok(const unp_view& v, const Want& want, std::string& why) {
  if (want.table_axis >= 0) {
    bool ok = (size_t)v.rank == want.shape.size();
    for (size_t d = 0; ok && d < want.shape.size(); ++d)
      ok = (int)d == want.table_axis ? v.shape[d] >= want.table_rows : v.shape[d] == want.shape[d];
    if (!ok) {
      std::vector<int64_t> t(want.shape);
      t[(size_t)want.table_axis] = want.table_rows;
      why = "the table view has shape " + shape_text(v.shape, (size_t)v.rank) + "; the extents ask for " +
            shape_text(t.data(), t.size()) + " (at least " + std::to_string(want.table_rows) + " along axis " +
            std::to_string(want.table_axis) + ")";
    }
    return ok;
  }
  if (shape_is(v, want.shape) || (!want.keepdim.empty() && shape_is(v, want.keepdim))) return true;
  why = "the view has shape " + shape_text(v.shape, (size_t)v.rank) + "; the extents ask for " +
        shape_text(want.shape.data(), want.shape.size()) +
        (want.keepdim.empty() ? std::string() : " or " + shape_text(want.keepdim.data(), want.keepdim.size()));
  return false;
}

bool view_empty(const unp_view& v) {
  for (int d = 0; d < v.rank; ++d)
    if (v.shape[d] == 0) return true;
  return false;
}

// Dense row-major from its base: every axis longer than one has the row-major stride.
bool row_major(const unp_view& v) {
  int64_t expect = 1;
  for (int d = v.rank - 1; d >= 0; --d) {
    if (v.shape[d] > 1 && v.stride[d] != expect) return false;
    expect *= v.shape[d];
  }
  return true;
}

// The gather index as the dense kernels read it: one id per position of the gathered axis, the
// other axes broadcast (stride 0), e.g. the embedding's [n, d] ids with strides [1, 0]
// (tests/kernel_parallel_gather_agrees.rs:80-84).
bool index_broadcast(const unp_view& v, int axis) {
  for (int d = 0; d < v.rank; ++d) {
    if (v.shape[d] <= 1) continue;
    if (d == axis ? v.stride[d] != 1 : v.stride[d] != 0) return false;
  }
  return true;
}

// Whether every view suits the pointer-launch kernels (dense row-major storage from the base).
bool views_dense(const unp_exec* x, const unp_view* v, size_t n, int64_t src_extent) {
  const unp_form& f = x->l.form;
  for (size_t b = 0; b < n; ++b) {
    if (view_empty(v[b])) continue;
    if (view_elem_bits(x->l, b) < 8 && v[b].base % 2 != 0) return false;  // a 4-bit view starting mid-byte
    if (f.kind == UNP_FORM_GATHER && !x->l.gx.plain) return false;  // one entry reads every layout
    if (f.kind == UNP_FORM_ELEMENTWISE && x->l.ew.permuted()) return false;  // the strided entry
    if (f.kind == UNP_FORM_GATHER && b < 2) {
      const int ax = x->l.scan_axis;
      if ((int)b == f.data_slot) {
        if (!row_major(v[b])) return false;
        // The dense kernels step A x src_extent rows: a table longer along a gathered axis
        // after the first needs the strides.
        if (ax > 0 && v[b].shape[ax] != src_extent) return false;
      } else if (!index_broadcast(v[b], ax)) {
        return false;
      }
      continue;
    }
    if (!row_major(v[b])) return false;
  }
  return true;
}

int32_t invalid(unp_error* err, const std::string& what) {
  set_error(err, UNP_INVALID_ARGUMENT, what);
  return UNP_INVALID_ARGUMENT;
}

// Checks shared by every launch of an executor: the device, the error, the timing state.
int32_t begin_launch(unp_exec* x, unp_error* err) {
  set_error(err, UNP_OK, "");
  x->t_first = true;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != x->device)
    return invalid(err, "the executor was created on another device");
  return UNP_OK;
}

// The strided entries' grid: a device-class constant (8 blocks of 256 per CU); blocks stride
// over the work and those past it exit.
uint32_t strided_grid(const unp_exec* x) { return (uint32_t)(x->cu_count * 8); }

size_t strided_entry(const unp_exec* x, int which) {
  for (size_t i = 0; i < x->l.entries.size(); ++i)
    if (x->l.entries[i].strided && which-- == 0) return i;
  return SIZE_MAX;
}

uint64_t view_ptr(const unp_view& v, size_t elem_bytes) { return v.data + (uint64_t)(v.base * (int64_t)elem_bytes); }

// A plain reduction (or the fused row fold) over storage images: one launch per output.
int32_t strided_reduction(unp_exec* x, const unp_view* v, const std::vector<int64_t>& ext, hipStream_t s,
                          unp_error* err) {
  const unp_form& f = x->l.form;
  const bool two = f.kind == UNP_FORM_ROW_REDUCE2;
  const uint32_t mask = x->l.axes_mask;
  long long outs = 1, count = 1;
  for (int32_t d = 0; d < f.rank; ++d) ((mask >> d) & 1u ? count : outs) *= ext[(size_t)d];
  if (outs == 0) return UNP_OK;
  const size_t eb = unp::kind_bytes(f.dtype);
  for (int o = 0; o < (two ? 2 : 1); ++o) {
    const unp_view& in = v[0];
    const unp_view& ov = v[1 + o];
    const bool keepdim = ov.rank == f.rank;
    long long in_str[UNP_MAX_RANK], out_str[UNP_MAX_RANK];
    for (int32_t a = 0, kept = 0; a < f.rank; ++a) {
      in_str[a] = in.stride[a];
      out_str[a] = 0;
      if (!((mask >> a) & 1u)) out_str[a] = keepdim ? ov.stride[a] : ov.stride[kept++];
    }
    unp::red_view_host d{};
    fill_red_view(ext, f.rank, mask, in_str, out_str, d);
    d.outs = outs;
    d.count = count;
    const size_t entry = strided_entry(x, o);
    uint64_t ip = view_ptr(in, eb), op = view_ptr(ov, eb);
    void* params[] = {&ip, &op, &d};
    const uint32_t grid = strided_grid(x);
    const int32_t rc = launch(x, entry, grid, params, s, err);
    if (rc != UNP_OK) return rc;
  }
  return UNP_OK;
}

// A scan over storage images: one lane per column, the scanned axis walked through its strides.
int32_t strided_scan(unp_exec* x, const unp_view* v, const std::vector<int64_t>& ext, hipStream_t s, unp_error* err) {
  const unp_form& f = x->l.form;
  const int ax = x->l.scan_axis;
  unp::scan_view_host d{};
  long long* const strs[2] = {d.cin, d.cout};
  long long cols = 1;
  for (int a = 0; a < f.rank; ++a) {
    if (a == ax) continue;
    cols *= ext[(size_t)a];
    const long long st[2] = {v[0].stride[a], v[1].stride[a]};
    add_axis<2>(d.cext, strs, d.nc, ext[(size_t)a], st);
  }
  d.S = ext[(size_t)ax];
  d.sin = v[0].stride[ax];
  d.sout = v[1].stride[ax];
  d.cols = cols;
  if (cols == 0 || d.S == 0) return UNP_OK;
  const size_t eb = unp::kind_bytes(f.dtype);
  uint64_t ip = view_ptr(v[0], eb), op = view_ptr(v[1], eb);
  void* params[] = {&ip, &op, &d};
  return launch(x, strided_entry(x, 0), strided_grid(x), params, s, err);
}

// A gather over storage images: one lane per output element.
int32_t strided_gather(unp_exec* x, const unp_view* v, const std::vector<int64_t>& ext, int64_t raw_src,
                       hipStream_t s, unp_error* err) {
  const unp_form& f = x->l.form;
  if (!x->l.gx.plain) {
    const size_t NI = (size_t)x->l.gx.n_inputs;
    unp::gather_x_view_host d{};
    d.rank = f.rank;
    d.axis = x->l.scan_axis;
    d.outs = 1;
    for (int a = 0; a < f.rank; ++a) {
      d.ext[a] = ext[(size_t)a];
      d.ostr[a] = v[NI].stride[a];
      d.outs *= ext[(size_t)a];
      for (size_t k = 0; k < NI; ++k) d.istr[k][a] = v[k].stride[a];
    }
    std::vector<uint64_t> ptrs;
    for (size_t k = 0; k <= NI; ++k) {
      const int32_t kind = (int)k == x->l.gx.index_slot ? f.index_dtype : f.dtype;
      ptrs.push_back(view_ptr(v[k], unp::kind_bytes(kind)));
    }
    return launch_gather_x(x, ptrs, d, raw_src, s, err);
  }
  const unp_view& tv = v[f.data_slot == 0 ? 0 : 1];
  const unp_view& iv = v[f.data_slot == 0 ? 1 : 0];
  const unp_view& ov = v[2];
  unp::gather_view_host d{};
  d.rank = f.rank;
  d.axis = x->l.scan_axis;
  long long outs = 1;
  for (int a = 0; a < f.rank; ++a) {
    d.ext[a] = ext[(size_t)a];
    d.tstr[a] = tv.stride[a];
    d.istr[a] = iv.stride[a];
    d.ostr[a] = ov.stride[a];
    outs *= ext[(size_t)a];
  }
  d.outs = outs;
  if (outs == 0) return UNP_OK;
  const int64_t src = gather_src_extent(f, raw_src);
  if (src <= 0 && f.oob == UNP_OOB_CLAMP) return invalid(err, "a Clamp gather needs a source extent of at least 1");
  const size_t eb = unp::kind_bytes(f.dtype), ib = unp::kind_bytes(f.index_dtype);
  uint64_t tp = view_ptr(tv, eb), ip = view_ptr(iv, ib), op = view_ptr(ov, eb);
  int32_t e32 = (int32_t)src;
  uint32_t eu32 = (uint32_t)src;
  long long e64 = src;
  void* ext_arg = f.index_dtype == UNP_I32 ? (void*)&e32 : (f.index_dtype == UNP_U32 ? (void*)&eu32 : (void*)&e64);
  void* params[] = {&tp, &ip, &op, &d, ext_arg};
  return launch(x, strided_entry(x, 0), strided_grid(x), params, s, err);
}

// An elementwise op over storage images: input k's stride along output axis d is its view's
// stride along its axis perm[d].
int32_t strided_elementwise(unp_exec* x, const unp_view* v, const std::vector<int64_t>& ext, hipStream_t s,
                            unp_error* err) {
  const unp_form& f = x->l.form;
  const unp::ElementwiseExpr& ew = x->l.ew;
  const size_t NI = (size_t)ew.n_inputs;
  unp::gather_x_view_host d{};
  d.rank = f.rank;
  d.outs = 1;
  for (int a = 0; a < f.rank; ++a) {
    d.ext[a] = ext[(size_t)a];
    d.ostr[a] = v[NI].stride[a];
    d.outs *= ext[(size_t)a];
    for (size_t k = 0; k < NI; ++k) d.istr[k][a] = v[k].stride[ew.perms.empty() ? a : ew.perms[k][(size_t)a]];
  }
  std::vector<uint64_t> ptrs;
  for (size_t k = 0; k <= NI; ++k) ptrs.push_back(view_ptr(v[k], unp::kind_bytes(f.dtype)));
  return launch_elementwise_strided(x, ptrs, d, s, err);
}

// Whether buffer parameter b of a lowered form is one it writes (an output).
bool writes_buffer(const unp_exec* x, size_t b) {
  switch (x->l.form.kind) {
    case UNP_FORM_ROW_REDUCE2: return b == 1 || b == 2;
    case UNP_FORM_DEQUANT4: return b == 3;
    case UNP_FORM_DEQUANT_GEMM: return b == 4;
    default: {
      size_t nbuf = 0, nscal = 0;
      param_counts(x, nbuf, nscal);
      return b + 1 == nbuf;  // the output follows the inputs
    }
  }
}

// Whether the view's elements are pairwise distinct storage positions: with the axes of extent
// above one ordered by |stride|, each stride exceeds the span of the smaller ones.
bool view_injective(const unp_view& v) {
  std::vector<std::pair<int64_t, int64_t>> ax;  // (|stride|, extent)
  for (int d = 0; d < v.rank; ++d)
    if (v.shape[d] > 1) ax.push_back({v.stride[d] < 0 ? -v.stride[d] : v.stride[d], v.shape[d]});
  std::sort(ax.begin(), ax.end());
  int64_t span = 0;
  for (const auto& a : ax) {
    if (a.first <= span) return false;
    span += a.first * (a.second - 1);
  }
  return true;
}

}  // namespace

// A form whose kernels read and write dense storage, over views some of which are not dense
// row-major: each such input view is packed into a dense copy the executor owns, the form's
// pointer launch runs on the copies, and a staged output is unpacked into its view afterwards
// (views.hip).  Elements outside the views are never touched.  An output view must not name an
// element twice.
static int32_t staged_launch(unp_exec* x, const unp_view* v, size_t n, const int64_t* scalars, size_t nscalars,
                             void* stream, unp_error* err) {
  int32_t rc = begin_launch(x, err);
  if (rc != UNP_OK) return rc;
  auto is_out = [&](size_t b) { return writes_buffer(x, b); };
  if (x->stage.size() < n) {
    x->stage.resize(n, nullptr);
    x->stage_cap.resize(n, 0);
  }
  std::vector<unp_arg> args(n + nscalars);
  std::vector<char> staged(n, 0);
  for (size_t b = 0; b < n; ++b) {
    const int bits = view_elem_bits(x->l, b);
    args[b].is_buffer = 1;
    const bool dense = view_empty(v[b]) || (row_major(v[b]) && (bits >= 8 || v[b].base % 2 == 0));
    if (dense) {
      args[b].value = v[b].data + (uint64_t)(v[b].base * bits / 8);
      continue;
    }
    if (is_out(b) && !view_injective(v[b]))
      return invalid(err, "buffer " + std::to_string(b) + ": an output view that names an element twice");
    const size_t bytes = (unp::view_stage_bytes(v[b], bits) + 255) & ~(size_t)255;
    if (x->stage_cap[b] < bytes) {
      if (x->stage[b]) hipFree(x->stage[b]);
      x->stage[b] = nullptr;
      x->stage_cap[b] = 0;
      const hipError_t e = hipMalloc(&x->stage[b], bytes);
      if (e != hipSuccess) return hip_fail(err, "hipMalloc(staged view)", e);
      x->stage_cap[b] = bytes;
    }
    if (!is_out(b) && (rc = unp::view_stage_in(v[b], bits, x->stage[b], stream, err)) != UNP_OK) return rc;
    args[b].value = (uint64_t)x->stage[b];
    staged[b] = 1;
  }
  for (size_t i = 0; i < nscalars; ++i) {
    args[n + i].is_buffer = 0;
    args[n + i].value = (uint64_t)scalars[i];
  }
  if ((rc = unp_hip_exec_launch(x, args.data(), args.size(), stream, err)) != UNP_OK) return rc;
  for (size_t b = 0; b < n; ++b)
    if (staged[b] && is_out(b) && (rc = unp::view_stage_out(x->stage[b], v[b], view_elem_bits(x->l, b), stream, err)) != UNP_OK)
      return rc;
  return UNP_OK;
}

extern "C" int32_t unp_hip_exec_launch_views(unp_exec* x, const unp_view* views, size_t nviews,
                                             const int64_t* scalars, size_t nscalars, void* stream,
                                             unp_error* err) {
  if (!x) return invalid(err, "null executor");
  if ((nviews && !views) || (nscalars && !scalars)) return invalid(err, "null views or scalars");
  const unp_form& f = x->l.form;
  size_t nbuf = 0, nscal = 0;
  param_counts(x, nbuf, nscal);
  if (nviews != nbuf || nscalars != nscal)
    return invalid(err, "expected " + std::to_string(nbuf) + " views and " + std::to_string(nscal) + " scalars, got " +
                            std::to_string(nviews) + " and " + std::to_string(nscalars));
  // The extents: the leading scalars, I32 as the KernelFn declares them.
  const size_t n_ext = f.kind == UNP_FORM_ROW_REDUCE ? (size_t)x->l.rr.rank
                       : f.kind == UNP_FORM_GATHER   ? (size_t)f.rank
                                                     : nscal;
  std::vector<int64_t> ext(n_ext);
  for (size_t i = 0; i < n_ext; ++i) {
    ext[i] = low_i32(scalars[i]);
    if (ext[i] < 0) return invalid(err, "extent n" + std::to_string(i) + " is negative");
  }
  const std::vector<Want> want = wanted_shapes(x, ext, scalars);
  if (want.size() != nbuf) return invalid(err, "unknown form");
  for (size_t b = 0; b < nviews; ++b) {
    const unp_view& v = views[b];
    const std::string at = "buffer " + std::to_string(b) + ": ";
    if (v.rank < 0 || v.rank > UNP_MAX_RANK) return invalid(err, at + "rank out of range");
    std::string why;
    if (!shape_ok(v, want[b], why)) return invalid(err, at + why);
    if (view_empty(v)) continue;
    // Every element the view names must lie at or above the storage start, and its offsets must
    // stay well inside the kernels' 64-bit index arithmetic.
    const int bits = view_elem_bits(x->l, b);
    __int128 lo = v.base, hi = v.base;
    for (int d = 0; d < v.rank; ++d) {
      const __int128 span = (__int128)v.stride[d] * (v.shape[d] - 1);
      (span < 0 ? lo : hi) += span;
    }
    if (lo < 0) return invalid(err, at + "the view reaches below its storage (base plus its negative strides < 0)");
    if (hi > ((__int128)1 << 60)) return invalid(err, at + "the view's offsets exceed 2^60 elements");
    if (bits < 8 && writes_buffer(x, b)) return invalid(err, at + "a 4-bit output view");
    if (!v.data) return invalid(err, at + "null storage");
  }
  const int64_t raw_src = f.kind == UNP_FORM_GATHER ? scalars[f.rank] : 0;
  const int64_t src = f.kind == UNP_FORM_GATHER ? gather_src_extent(f, raw_src) : 0;
  if (views_dense(x, views, nviews, src)) {
    std::vector<unp_arg> args(nviews + nscalars);
    for (size_t b = 0; b < nviews; ++b) {
      const int bits = view_elem_bits(x->l, b);
      args[b].is_buffer = 1;
      args[b].value = views[b].data + (uint64_t)(views[b].base * bits / 8);
    }
    for (size_t i = 0; i < nscalars; ++i) {
      args[nviews + i].is_buffer = 0;
      args[nviews + i].value = (uint64_t)scalars[i];
    }
    return unp_hip_exec_launch(x, args.data(), args.size(), stream, err);
  }
  // Some view is transposed, strided, reversed or broadcast: the forms with a strided entry read
  // through the strides; the others stage those views through dense copies.
  const bool plain_reduction = (f.kind == UNP_FORM_REDUCTION && x->l.rx.plain) || f.kind == UNP_FORM_ROW_REDUCE2;
  const bool plain_scan = f.kind == UNP_FORM_SCAN && x->l.rx.plain;
  if (!plain_reduction && !plain_scan && f.kind != UNP_FORM_GATHER && f.kind != UNP_FORM_ELEMENTWISE)
    return staged_launch(x, views, nviews, scalars, nscalars, stream, err);
  const int32_t rc = begin_launch(x, err);
  if (rc != UNP_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (plain_reduction) return strided_reduction(x, views, ext, s, err);
  if (f.kind == UNP_FORM_ELEMENTWISE) return strided_elementwise(x, views, ext, s, err);
  if (f.kind == UNP_FORM_SCAN) return strided_scan(x, views, ext, s, err);
  return strided_gather(x, views, ext, raw_src, s, err);
}

extern "C" int32_t unp_hip_exec_launch(unp_exec* x, const unp_arg* args, size_t nargs, void* stream,
                                       unp_error* err) {
  if (!x) {
    set_error(err, UNP_INVALID_ARGUMENT, "null executor");
    return UNP_INVALID_ARGUMENT;
  }
  const int32_t rc = begin_launch(x, err);
  if (rc != UNP_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  switch (x->l.form.kind) {
    case UNP_FORM_REDUCTION:
    case UNP_FORM_ROW_REDUCE2:
      return run_reduction(x, args, nargs, s, err);
    case UNP_FORM_SCAN:
      return run_scan(x, args, nargs, s, err);
    case UNP_FORM_GATHER:
      return run_gather(x, args, nargs, s, err);
    case UNP_FORM_ROW_REDUCE:
      return run_row_reduce(x, args, nargs, s, err);
    case UNP_FORM_DEQUANT4:
      return run_dequant(x, args, nargs, s, err);
    case UNP_FORM_DEQUANT_GEMM:
      return run_dequant_gemm(x, args, nargs, s, err);
    case UNP_FORM_ELEMENTWISE:
      return run_elementwise(x, args, nargs, s, err);
    default:
      set_error(err, UNP_UNSUPPORTED_KERNEL, "unknown form");
      return UNP_UNSUPPORTED_KERNEL;
  }
}

namespace unp {

int32_t exec_launch_in(unp_exec* x, const unp_arg* args, size_t nargs, void* stream, void* scratch, size_t cap,
                       unp_error* err) {
  if (!x || !scratch) {
    set_error(err, UNP_INVALID_ARGUMENT, "null executor or scratch");
    return UNP_INVALID_ARGUMENT;
  }
  const Scratch sc{scratch, cap};
  x->fixed = &sc;
  const int32_t rc = unp_hip_exec_launch(x, args, nargs, stream, err);
  x->fixed = nullptr;
  return rc;
}

}  // namespace unp
