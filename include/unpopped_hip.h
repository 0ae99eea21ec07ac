/*
 * unpopped-hip: an MI355X (gfx950) backend for the Unpopped kernel generator, as a C ABI.
 *
 * The reference (EvansLaboratories/Unpopped 0.56.5) defines two seams a device backend
 * implements, both Rust traits:
 *
 *   trait Backend   crates/unpopped/src/backend.rs:668-807   (name, provider, lower,
 *                   lower_kernel, supports_dtype, total_integer_ops, effective_count_width,
 *                   lower_variants)
 *   trait Compiler  crates/unpopped/src/jit.rs:271-285       (compile, artifact_kind)
 *
 * and stops before the launch (no reference source writes a launch: docs/PATENT-SWEEP.md
 * :265-272).  This library is the HIP side of both seams plus the launch layer a consumer
 * needs: a thin FFI over the HIP runtime (hipModuleLoadData, hipModuleLaunchKernel,
 * hipMalloc, hipEvent*) and a prepared-kernel executor that owns the look-back / partial
 * workspaces and picks the launch geometry from the device.
 *
 * Conventions (backend.rs:703-707, jit.rs:397-401): every entry point returns a status
 * code and never aborts; a refusal is a typed code plus a diagnostic string that is for
 * people, not for matching.  Everything the library allocates is released by the
 * matching unp_*_free / _destroy call.  Handles are not thread-safe; one caller at a time.
 */
#ifndef UNPOPPED_HIP_H
#define UNPOPPED_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------
 * Status codes.  1..6 mirror LowerError (crates/unpopped/src/backend.rs:386-440) in
 * declaration order; the rest are this library's own.
 * ------------------------------------------------------------------------------------- */
enum unp_status {
  UNP_OK = 0,
  UNP_UNSUPPORTED_DTYPE = 1,      /* LowerError::UnsupportedDtype      backend.rs:388 */
  UNP_UNSUPPORTED_SCHEDULE = 2,   /* LowerError::UnsupportedSchedule   backend.rs:396 */
  UNP_UNSUPPORTED_OP = 3,         /* LowerError::UnsupportedOp         backend.rs:402 */
  UNP_UNSUPPORTED_PLAN_SHAPE = 4, /* LowerError::UnsupportedPlanShape  backend.rs:408 */
  UNP_INADMISSIBLE_PLAN = 5,      /* LowerError::InadmissiblePlan      backend.rs:424 */
  UNP_UNSUPPORTED_KERNEL = 6,     /* LowerError::UnsupportedKernel     backend.rs:436 */
  UNP_LIFT_DECLINE = 10,          /* LiftDecline (kernel_lift.rs:48-85); detail names it */
  UNP_COMPILE_ERROR = 20,         /* Compiler::compile Err(String)     jit.rs:278 */
  UNP_HIP_ERROR = 30,             /* a HIP runtime call failed; detail has hipGetErrorString */
  UNP_STALLED = 31,               /* a launch gave up waiting for another block (no reference
                                     counterpart: unp_hip_exec_check) */
  UNP_INVALID_ARGUMENT = 40,      /* a launch argument does not fit the kernel's interface */
  UNP_PARSE_ERROR = 50            /* kernel JSON text that is not a KernelFn */
};

typedef struct unp_error {
  int32_t code;
  char detail[512];
} unp_error;

/* ---------------------------------------------------------------------------------------
 * Element kinds: the reference's ElementKind (crates/unpopped-vocab/src/element.rs:1052)
 * in declaration order; the JSON form uses the variant names (crates/unpopped/src/text.rs:56).
 * ------------------------------------------------------------------------------------- */
enum unp_element_kind {
  UNP_F16 = 0, UNP_BF16 = 1, UNP_F32 = 2, UNP_F32_STRICT = 3, UNP_F64 = 4,
  UNP_I8 = 5, UNP_I16 = 6, UNP_U8 = 7, UNP_U16 = 8, UNP_I32 = 9, UNP_I64 = 10, UNP_BOOL = 11,
  UNP_FP8_E4M3FN = 12, UNP_FP8_E4M3FNUZ = 13, UNP_FP8_E5M2 = 14, UNP_F8_E8M0 = 15,
  UNP_F8_E6M2 = 16, UNP_FP8_E5M2FNUZ = 17, UNP_I4 = 18, UNP_U4 = 19, UNP_B1 = 20,
  UNP_COMPLEX64 = 21, UNP_COMPLEX128 = 22, UNP_U32 = 23, UNP_U64 = 24,
  UNP_F4_E2M1 = 25, UNP_F6_E2M3 = 26, UNP_F6_E3M2 = 27
};

/* DtypeSupport (backend.rs:645-655). */
enum unp_dtype_support { UNP_SUPPORTED = 0, UNP_UNSUPPORTED = 1, UNP_NOT_EXPRESSIBLE = 2 };

/* ArtifactKind (crates/unpopped/src/jit.rs:139-152); this compiler answers HipCodeObject. */
enum unp_artifact_kind {
  UNP_ARTIFACT_PTX = 0, UNP_ARTIFACT_CUBIN = 1, UNP_ARTIFACT_HIP_CODE_OBJECT = 2,
  UNP_ARTIFACT_SPIRV = 3, UNP_ARTIFACT_STUB = 4
};

/* ---------------------------------------------------------------------------------------
 * Backend seam (trait Backend, backend.rs:668-807).
 * ------------------------------------------------------------------------------------- */

/* Backend::name (backend.rs:671): "hip". */
const char* unp_hip_name(void);
/* Backend::provider (backend.rs:681): "unpopped-hip". */
const char* unp_hip_provider(void);
/* Backend::total_integer_ops (backend.rs:682-694): 1.  Integer Div, Shl, Shr and ConstInt at the
 * I32, I64, U32 and U64 compute dtypes are spelled by the total rule of
 * docs/int-div-shift-semantics.md (rules 1-3): a zero divisor gives the dividend, so does signed
 * MIN / -1; a shift count is read as unsigned bits modulo 32 (modulo 64 for a 64-bit type); Shl
 * wraps and Shr is arithmetic on signed types, logical on unsigned ones; Add, Sub and Mul wrap. */
int32_t unp_hip_total_integer_ops(void);
/* Backend::supports_dtype (backend.rs:779): one of unp_dtype_support for an element kind on
 * a target id such as "rocm:gfx950" (crates/unpopped-vocab/src/target.rs:188). */
int32_t unp_hip_supports_dtype(int32_t kind, const char* target);

/* GeneratedKernel (backend.rs:105-193): name, source and the launch interface as JSON. */
typedef struct unp_generated unp_generated;
const char* unp_generated_name(const unp_generated* g);
const char* unp_generated_source(const unp_generated* g);
const char* unp_generated_interface_json(const unp_generated* g);
/* FNV-1a 64 over the source text (crates/unpopped/src/revision.rs). */
uint64_t unp_generated_revision_hash(const unp_generated* g);
void unp_generated_free(unp_generated* g);

/* A lowering request in the backend's own terms: the launched reduction, scan, gather,
 * sub-byte dequant and fused row-reduce forms that lower_kernel recognises in a KernelFn.
 * Fields not used by a form are ignored. */
enum unp_form_kind {
  UNP_FORM_REDUCTION = 0, /* Access::Reduction, launched (kernel_lift/block_reduce.rs:50) */
  UNP_FORM_SCAN = 1,      /* Access::Scan, launched (kernel_lift/scan_launched.rs:54) */
  UNP_FORM_GATHER = 2,    /* ReadIndex::Indexed gather (kernel_lift/gather.rs:35) */
  UNP_FORM_DEQUANT4 = 3,  /* U4/I4 x f16 scale x 4-bit zero -> bf16 (tests/support/dequant.rs) */
  UNP_FORM_ROW_REDUCE2 = 4, /* two folds of each row read once (Sum and Max: softmax prologue) */
  UNP_FORM_ROW_REDUCE = 5,  /* Access::RowReduce: staged row folds, then a full-width epilogue
                               (kernel_lift/row_reduce.rs:31, row_reduce_launched.rs:47); its
                               expressions come only through unp_hip_lower_kernel */
  UNP_FORM_DEQUANT_GEMM = 6, /* the dequantizing GEMM (tests/support/dequant.rs:104-181): U4/I4
                               weights, I32 zero and scale per group, I32 or I8 activations,
                               I32 out, all wrapping */
  UNP_FORM_ELEMENTWISE = 7  /* Access::Elementwise, launched (kernel_lift.rs:96-153): a body over
                               n inputs read at the output coordinate, each optionally through an
                               axis permutation; its body comes only through unp_hip_lower_kernel */
};
/* ReduceOp subset (crates/unpopped/src/ir.rs:1700-1735).  And/Or/Xor fold integers bitwise;
 * MaxNum/MinNum ignore NaN (a run of only NaN gives NaN); the reference lifts these five as
 * sequential reductions only (kernel_lift.rs:763-800, block_reduce.rs:97-133). */
enum unp_reduce_op {
  UNP_OP_SUM = 0, UNP_OP_PROD = 1, UNP_OP_MAX = 2, UNP_OP_MIN = 3, UNP_OP_MEAN = 4,
  UNP_OP_AND = 5, UNP_OP_OR = 6, UNP_OP_XOR = 7, UNP_OP_MAXNUM = 8, UNP_OP_MINNUM = 9
};
/* OobPolicy (ir.rs:2582). */
enum unp_oob_policy { UNP_OOB_SKIP = 0, UNP_OOB_ZEROFILL = 1, UNP_OOB_CLAMP = 2 };
/* The schedule a form lowers to.  SERIAL is the serial lift's own order (one lane per output of a
 * reduction, per column of a scan): the bits of the sequential fold the reference's
 * Schedule::Reduction and Schedule::Scan { block: false } name (plan/types.rs:30-75).  DEVICE is
 * this backend's device-class schedule.  FIXED is the device schedule with every float
 * association fixed by the launch's tiling, so a float result is the same on every launch (the
 * reference's launched lifts fix theirs by geometry, kernel_lift/scan_launched.rs:19-26): a
 * float scan's look-back (with or without a pre-map) folds tile aggregates in a fixed grouping;
 * every other form's device schedule is already fixed and lowers unchanged.  A float scan's
 * DEVICE look-back folds however far each look-back walked, which timing decides: its bits can
 * change from launch to launch, so unp_hip_lower_kernel lowers a lifted float scan on FIXED and
 * DEVICE is only a Nondeterministic variant.  Forms whose every schedule gives the same bits
 * (the gather, the dequants, integer folds) lower the same kernels whichever is asked. */
enum unp_schedule { UNP_SCHEDULE_DEVICE = 0, UNP_SCHEDULE_SERIAL = 1, UNP_SCHEDULE_FIXED = 2 };
/* VariantFidelity (backend.rs:204-309) in declaration order: a variant's bits against the cell's
 * default lowering (here the SERIAL schedule, the sequential fold's bits). */
enum unp_fidelity {
  UNP_BIT_IDENTICAL = 0,
  UNP_DETERMINISTICALLY_DIVERGENT = 1,
  UNP_NONDETERMINISTIC = 2,
  UNP_MORE_PRECISE = 3
};

typedef struct unp_form {
  int32_t kind;        /* unp_form_kind */
  int32_t dtype;       /* element kind of the data (gather: of the table) */
  int32_t rank;        /* input rank (reduction/scan), output rank (gather); 2 for dequant */
  int32_t op0, op1;    /* unp_reduce_op; op1 only for UNP_FORM_ROW_REDUCE2 */
  int32_t reduced_from;/* reduction: first reduced axis; axes reduced_from..rank-1 fold */
  int32_t exclusive;   /* scan */
  int32_t reverse;     /* scan */
  int32_t index_dtype; /* gather: I32, I64 or U32 */
  int32_t oob;         /* gather: unp_oob_policy */
  int32_t data_slot;   /* gather: which input (0 or 1) is the table; the other is the index */
  int32_t q_kind;      /* dequant: U4 or I4 weights */
  int32_t z_kind;      /* dequant: U4 or I4 zero points */
  int32_t group;       /* dequant: columns per scale/zero group */
  int32_t out_kind;    /* dequant: Bf16 */
  uint32_t axes_mask;  /* reduction: the reduced axes, bit d = axis d (ReductionShape::new,
                          kernel_lift.rs:854-870); 0 means axes reduced_from..rank-1.
                          scan: the scanned axis as its one bit; 0 means the innermost axis.
                          gather: the gathered axis as its one bit; 0 means axis 0 */
  int32_t schedule;    /* unp_schedule; 0 (DEVICE) for every form lowered before it existed */
} unp_form;

/* Lower one form to HIP source (the work Backend::lower_kernel does once it has recognised
 * the lifted kernel, and Backend::lower does for a plan the binding maps to a form).  *out is
 * owned by the caller (unp_generated_free).  A schedule a form does not have is
 * UNP_UNSUPPORTED_SCHEDULE. */
int32_t unp_hip_lower_form(const unp_form* form, unp_generated** out, unp_error* err);

/* Variant (backend.rs:313-353): a tag, the form to lower (unp_hip_lower_form) and its fidelity
 * against the cell's default lowering, the SERIAL schedule. */
typedef struct unp_variant {
  char tag[32];
  int32_t fidelity; /* unp_fidelity */
  unp_form form;
  char launch_note[256];
} unp_variant;
/* Backend::lower_variants (backend.rs:786-807): every schedule this backend has for the form's
 * cell, the default (SERIAL) first, then the reproducible ones, then a Nondeterministic one.  Fills up to `cap` entries of `out` and sets *count to the
 * number there are; a form with no lowering is refused as unp_hip_lower_form refuses it. */
int32_t unp_hip_form_variants(const unp_form* form, unp_variant* out, size_t cap, size_t* count, unp_error* err);

/* Backend::lower_kernel (backend.rs:726-737): lower a kernel-layer KernelFn, given as the JSON
 * serde writes for the reference's `KernelFn` (crates/unpopped/src/kernel.rs:1223-1250; element
 * kinds by variant name, crates/unpopped/src/text.rs:56-91).  The kernel is recognised as one of
 * the lifts below (or the two kernels this backend authors) by lifting each candidate form its
 * signature admits and comparing the trees; anything else is UNP_UNSUPPORTED_KERNEL, and text that
 * is not a KernelFn is UNP_PARSE_ERROR.  The interface JSON carries the kernel's declared launch
 * and parameters (KernelInterface::of, kernel_interface.rs:237-262) beside the HIP launch.  A
 * float scan lowers the FIXED schedule (reproducible bits); every other form its DEVICE one. */
int32_t unp_hip_lower_kernel(const char* kernel_json, unp_generated** out, unp_error* err);

/* ---------------------------------------------------------------------------------------
 * The lifts, restated (each returns the KernelFn as JSON in *json, freed with unp_free_str;
 * a refusal is UNP_LIFT_DECLINE with the LiftDecline variant in err->detail).  block = grid = 0
 * asks for the serial lift; otherwise the launched lift on grid blocks of block threads.
 * ------------------------------------------------------------------------------------- */

/* lift_reduction_opdef (kernel_lift.rs:447-484) / lift_reduction_opdef_launched
 * (kernel_lift/block_reduce.rs:50-93) of OpDef::reduction_axes(name, 1, [dtype], Input(0), op,
 * axes, keepdim) (ir.rs:3186-3214): axes_mask bit d reduces axis d, 0 is the last axis. */
int32_t unp_lift_reduction(const char* name, int32_t dtype, int32_t rank, int32_t op, uint32_t axes_mask,
                           int32_t keepdim, uint32_t block, uint32_t grid, char** json, unp_error* err);
/* The same lifts of an OpDef::reduction with n_inputs inputs, a pre-map body over Input(0..n) and
 * a fused post over Reduced(0) (kernel_lift.rs:807-831, :910-1003; block_reduce.rs:292-307), both
 * as ScalarExpr JSON; post_json NULL (or `{"Reduced":0}`) is the identity post. */
int32_t unp_lift_reduction_x(const char* name, int32_t dtype, int32_t rank, int32_t op, uint32_t axes_mask,
                             int32_t keepdim, int32_t n_inputs, const char* body_json, const char* post_json,
                             uint32_t block, uint32_t grid, char** json, unp_error* err);
/* lift_scan_opdef (kernel_lift.rs:504-519) / lift_scan_opdef_launched (kernel_lift/scan_launched.rs
 * :54-102) of OpDef::scan_simple (ir.rs:3422-3441): identity pre-map, no post. */
int32_t unp_lift_scan(const char* name, int32_t dtype, int32_t rank, int32_t op, int32_t axis, int32_t exclusive,
                      int32_t reverse, uint32_t block, uint32_t grid, char** json, unp_error* err);
/* The same lifts of an Access::Scan with n_inputs inputs, a pre-map over Input(0..n) and a fused
 * post over Reduced(0) (the prefix rounded once) and Input(0..n) (the elements at the position)
 * (kernel_lift.rs:530-602, :658-690; scan_launched.rs:140-160), both as ScalarExpr JSON; post_json
 * NULL (or `{"Reduced":0}`) is the identity post. */
int32_t unp_lift_scan_x(const char* name, int32_t dtype, int32_t rank, int32_t op, int32_t axis, int32_t exclusive,
                        int32_t reverse, int32_t n_inputs, const char* pre_json, const char* post_json,
                        uint32_t block, uint32_t grid, char** json, unp_error* err);
/* lift_gather_opdef (kernel_lift/gather.rs:35-55) / lift_gather_opdef_launched (kernel_lift.rs
 * :183-191) of OpDef::gather(name, [dtype, index_dtype], axis, oob, index_dtype) (ir.rs:3838-3855);
 * OpDef::embedding is axis 0 with ZeroFill (ir.rs:3884-3886). */
int32_t unp_lift_gather(const char* name, int32_t dtype, int32_t rank, int32_t index_dtype, int32_t axis,
                        int32_t oob, uint32_t block, uint32_t grid, char** json, unp_error* err);
/* The gather lift in general (kernel_lift/gather.rs:35-101): n_inputs (2..8) inputs, input
 * index_slot the integer index, input data_slot the gathered one, the others read at the output
 * coordinate, and body_json (a ScalarExpr over Input(0..n_inputs), constants allowed) stored at the
 * output coordinate. */
int32_t unp_lift_gather_x(const char* name, int32_t dtype, int32_t rank, int32_t index_dtype, int32_t axis,
                          int32_t oob, int32_t n_inputs, int32_t data_slot, int32_t index_slot, const char* body_json,
                          uint32_t block, uint32_t grid, char** json, unp_error* err);
/* lift_elementwise_opdef (kernel_lift.rs:96-130) / lift_elementwise_opdef_launched (:145-153): n_inputs
 * (1..8) inputs of dtype read at the loop counters, body_json (a ScalarExpr over Input(0..n_inputs),
 * constants allowed) stored at the output coordinate.  perms: NULL for identity reads, else
 * n_inputs x rank axis indices, row k the View::Permute of input k (iteration axis d reads the
 * input's axis perms[k * rank + d], counter_place, kernel_lift.rs:315-324); block and grid 0 for
 * the serial lift. */
int32_t unp_lift_elementwise(const char* name, int32_t dtype, int32_t rank, int32_t n_inputs, const char* body_json,
                             const int32_t* perms, uint32_t block, uint32_t grid, char** json, unp_error* err);
/* No reference lift: the fused two-fold row reduction (softmax prologue) this backend authors,
 * each fold exactly a serial lifted reduction's; launched, rows grid-strided. */
int32_t unp_kernel_row_reduce2(const char* name, int32_t dtype, int32_t op0, int32_t op1, uint32_t block,
                               uint32_t grid, char** json, unp_error* err);
/* No reference lift: the int4 dequant this backend authors after the dequant-GEMM fixture
 * (crates/unpopped/tests/support/dequant.rs:58-143): out[r, c] = Bf16_rne((q - z) * s) with a U4/I4
 * weight, a U4/I4 zero point and an F16 scale per `group` columns. */
int32_t unp_kernel_dequant4(const char* name, int32_t q_kind, int32_t z_kind, int32_t group, uint32_t block,
                            uint32_t grid, char** json, unp_error* err);
/* No reference lift: the dequantizing GEMM of the reference's fixture
 * (crates/unpopped/tests/support/dequant.rs:104-181; docs/options-u9b-subbyte-dequant.md:28-30)
 * with the extents as scalars:
 * out[r][c] = sum over k of (w[r][k] - zero[r][k / group]) * scale[r][k / group] * x[k][c], every
 * operation an I32 that wraps.  Buffers w (w_kind U4 or I4, R x K, two to a byte, low nibble
 * first), zero and scale (I32, R x ceil(K / group)), x (x_kind I32 as in the reference, or I8;
 * K x C), out (I32, R x C); scalars n0 = R, n1 = K, n2 = C.  block = grid = 0: the serial
 * kernel; otherwise rows grid-strided.  The recognised form carries w_kind in q_kind, x_kind in
 * dtype and the group in group. */
int32_t unp_kernel_dequant_gemm(const char* name, int32_t w_kind, int32_t x_kind, int32_t group, uint32_t block,
                                uint32_t grid, char** json, unp_error* err);

/* lift_row_reduce_opdef (crates/unpopped/src/kernel_lift/row_reduce.rs:31-49) and, with a
 * launch, lift_row_reduce_opdef_launched (kernel_lift/row_reduce_launched.rs:47-86) of the
 * Access::RowReduce op (crates/unpopped/src/ir.rs:2114-2125, OpDef::row_reduce ir.rs:3268):
 * `stages_json` is the JSON array of its ReduceStage {pre, op} (ir.rs:2049), `epilogue_json` the
 * epilogue ScalarExpr, both over Input(k) and Reduced(t) leaves; `n_inputs` inputs of `dtype`
 * (F32 or F64) and rank `rank`.  block = grid = 0 lifts the serial kernel. */
int32_t unp_lift_row_reduce(const char* name, int32_t dtype, int32_t rank, int32_t n_inputs,
                            const char* stages_json, const char* epilogue_json, uint32_t block,
                            uint32_t grid, char** json, unp_error* err);

/* ---------------------------------------------------------------------------------------
 * Compiler seam (trait Compiler, jit.rs:271-285), through hipRTC for gfx950.
 * ------------------------------------------------------------------------------------- */

/* Compiler::compile (jit.rs:278): source -> code-object bytes.  max_compile_ms = 0 means no
 * budget; a compile that overruns a nonzero budget is an error.  *bytes is freed with
 * unp_free_bytes, *diag (the compiler log, may be NULL) with unp_free_str. */
int32_t unp_hip_compile(const char* source, const char* entry, uint32_t max_compile_ms,
                        uint8_t** bytes, size_t* len, char** diag);
/* Compiler::artifact_kind (jit.rs:282): UNP_ARTIFACT_HIP_CODE_OBJECT. */
int32_t unp_hip_artifact_kind(void);
void unp_free_bytes(uint8_t* p);
void unp_free_str(char* s);

/* ---------------------------------------------------------------------------------------
 * HIP runtime FFI (the consumer's launch layer; no reference counterpart by design).
 * ------------------------------------------------------------------------------------- */
typedef struct unp_module unp_module;
typedef struct unp_function unp_function;
typedef struct unp_event unp_event;

int32_t unp_hip_device_count(int32_t* count);
int32_t unp_hip_set_device(int32_t device);
/* gcnArchName (e.g. "gfx950:sramecc+:xnack-") and compute-unit count of the current device. */
int32_t unp_hip_device_info(char* arch, size_t arch_len, int32_t* cu_count);
int32_t unp_hip_module_load(const uint8_t* image, size_t len, unp_module** out, unp_error* err);
int32_t unp_hip_module_unload(unp_module* m);
int32_t unp_hip_get_function(unp_module* m, const char* name, unp_function** out, unp_error* err);
/* Launch with a packed kernel-argument block (the layout the interface JSON states). */
int32_t unp_hip_launch(unp_function* f, const uint32_t grid[3], const uint32_t block[3],
                       uint32_t shared_bytes, void* stream, const void* kernarg, size_t kernarg_size,
                       unp_error* err);
/* The same launch with `start` and `stop` recorded at the kernel's own dispatch timestamps
 * (hipExtModuleLaunchKernel), so unp_hip_event_elapsed_ms(start, stop) is the kernel's time without
 * the queueing around it, as a kernel trace shows it.  Either event may be null; grid x block must
 * stay below 2^32 in each dimension. */
int32_t unp_hip_launch_timed(unp_function* f, const uint32_t grid[3], const uint32_t block[3],
                             uint32_t shared_bytes, void* stream, const void* kernarg, size_t kernarg_size,
                             unp_event* start, unp_event* stop, unp_error* err);
int32_t unp_hip_malloc(void** p, size_t bytes);
int32_t unp_hip_free(void* p);
int32_t unp_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int32_t unp_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
int32_t unp_hip_memset(void* p, int32_t value, size_t bytes);
int32_t unp_hip_synchronize(void);
int32_t unp_hip_event_create(unp_event** e);
int32_t unp_hip_event_destroy(unp_event* e);
int32_t unp_hip_event_record(unp_event* e, void* stream);
int32_t unp_hip_event_synchronize(unp_event* e);
int32_t unp_hip_event_elapsed_ms(unp_event* start, unp_event* stop, float* ms);

/* ---------------------------------------------------------------------------------------
 * Prepared kernels: a lowered kernel compiled (in-process, compile-once per source) and
 * loaded on the current device, with the workspace its schedule needs.
 * ------------------------------------------------------------------------------------- */
typedef struct unp_exec unp_exec;

/* One launch argument, in the lowered KernelFn's parameter order: a buffer is a device
 * pointer, a scalar is an integer (the reference's extents are I32 scalars). */
typedef struct unp_arg {
  int32_t is_buffer;
  int32_t pad;
  uint64_t value; /* device address or scalar value */
} unp_arg;

int32_t unp_hip_exec_create(const unp_generated* g, unp_exec** out, unp_error* err);
int32_t unp_hip_exec_launch(unp_exec* e, const unp_arg* args, size_t nargs, void* stream,
                            unp_error* err);
/* One buffer as the reference's storage image (TypedBuffer, crates/unpopped/src/oracle/
 * buffers.rs:16-42; the C leg passes the same per buffer, unpopped-cpu-c/src/base.rs:65-103):
 * the device address of the allocation, the view's rank, shape and signed element strides, and
 * its base offset in elements.  Sub-byte kinds (U4, I4) count elements, two to a byte. */
#define UNP_MAX_RANK 8
typedef struct unp_view {
  uint64_t data;
  int32_t rank;
  int32_t pad;
  int64_t shape[UNP_MAX_RANK];
  int64_t stride[UNP_MAX_RANK];
  int64_t base;
} unp_view;

/* unp_hip_exec_launch with the buffers as storage images, in the KernelFn's parameter order
 * (views for the buffer parameters, then the scalars).  The shape is authoritative, as in the
 * reference's TypedBuffer: each view must have exactly the shape the extent scalars give its
 * parameter (a reduction's output: the kept extents, or the keepdim shape with the reduced axes
 * of extent 1; a gather's table: the output's extents except along the gathered axis, where it
 * holds at least src_extent rows), must not reach below its storage (base plus every negative
 * stride times its extent less one), and an output view must name each element once; anything else
 * is UNP_INVALID_ARGUMENT before anything launches.
 * Dense row-major views (any stride on an axis of extent one; a 4-bit view starting on a whole
 * byte; the gather index broadcast along every axis but the gathered one, e.g. [n, d] with strides
 * [1, 0], tests/kernel_parallel_gather_agrees.rs:80-84) launch the pointer kernels at data + base.
 * Any other view -- transposed, strided, negative strides, broadcast, a full-shape gather index --
 * is read and written through its strides by the reduction (plain body), fused row fold, scan,
 * gather and elementwise forms (their "strided" interface entries).  The row-reduce, pre-map
 * reduction, pre-map scan and dequant forms stage it: each such input view is packed into a dense
 * copy the executor owns (allocated on first use), the pointer kernels run on the copies, and a
 * staged output is unpacked into its view; elements outside the views are never touched.  The
 * storage behind a view is the caller's: every element the view names must lie inside it. */
int32_t unp_hip_exec_launch_views(unp_exec* e, const unp_view* views, size_t nviews, const int64_t* scalars,
                                  size_t nscalars, void* stream, unp_error* err);
/* No reference counterpart: it exists for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  unp_hip_exec_launch with every
 * workspace the executor would allocate (scan tile status and ticket counter, reduction partials and
 * counters, the dequant GEMM's repacked activations) taken from one static device array of
 * UNP_STATIC_SCRATCH_BYTES per GPU instead; the call allocates and frees nothing.  A launch whose
 * workspace does not fit is refused with UNP_INVALID_ARGUMENT before anything runs.  Each call
 * clears the part of the array it uses on its stream first; calls that overlap on one GPU share the
 * array and race, so a caller serialises them. */
#define UNP_STATIC_SCRATCH_BYTES (4u << 20)
int32_t unp_hip_exec_launch_static(unp_exec* e, const unp_arg* args, size_t nargs, void* stream, unp_error* err);
/* Kernel timing for reports (no reference counterpart): after this call every launch of `e` records
 * `start` at the beginning of its first kernel and `stop` at the end of its last, from the kernels'
 * own dispatch timestamps (hipExtModuleLaunchKernel), so unp_hip_event_elapsed_ms(start, stop) is
 * the launch's kernel time without the queueing gap around it.  NULL, NULL restores plain launches;
 * the events must stay alive while they are set. */
int32_t unp_hip_exec_set_timing(unp_exec* e, unp_event* start, unp_event* stop);
/* Bounded waits (no reference counterpart: the reference's CPU launches never wait on another
 * thread).  A kernel that waits for another block of its launch -- a scan tile for its
 * predecessors' status, a full or column reduction's folding block for the other blocks' partials,
 * a staged scan's waves for their tile's look-back -- gives up once one wait has lasted `wait_us`
 * microseconds of the device's wall clock (default 1 s; 0 gives up at the first unanswered probe),
 * goes on with the fold's identity in place of the missing value, and counts the give-up in a word
 * of the executor.  Every block still finishes, so a lost predecessor ends the launch with wrong
 * outputs instead of hanging the device.  unp_hip_exec_check waits for the device and returns
 * UNP_STALLED, and clears the count, when any launch of `e` since the last check gave up; else
 * UNP_OK. */
int32_t unp_hip_exec_set_wait_limit(unp_exec* e, uint32_t wait_us);
int32_t unp_hip_exec_check(unp_exec* e, unp_error* err);
/* The last launch's geometry and chosen entry point (for reports). */
int32_t unp_hip_exec_last_launch(const unp_exec* e, uint32_t grid[3], uint32_t block[3],
                                 char* entry, size_t entry_len);
void unp_hip_exec_destroy(unp_exec* e);

#ifdef __cplusplus
}
#endif

#endif /* UNPOPPED_HIP_H */
