/*
 * CPU oracle for the unpopped-hip hot path.  TEST INFRASTRUCTURE ONLY: the parity tests, the
 * smoke check and the benchmark's CPU-baseline leg call it as the checker.  No product code
 * links or calls it.
 *
 * A plain-C restatement of the reference's semantics for the forms the HIP backend lowers
 * (EvansLaboratories/Unpopped 0.56.5, Rust, which has no toolchain here and cannot be
 * built or imported).  Each function cites the reference file:line it follows; the pinning
 * of each one (golden vectors, closed forms, library routines, brute force) lives in
 * tests/test_oracle.py.
 */
#ifndef UNPOPPED_ORACLE_H
#define UNPOPPED_ORACLE_H

#include <stdint.h>

/* ReduceOp subset and OobPolicy codes (as include/unpopped_hip.h). */
enum {
  ORC_SUM = 0, ORC_PROD = 1, ORC_MAX = 2, ORC_MIN = 3, ORC_MEAN = 4,
  ORC_AND = 5, ORC_OR = 6, ORC_XOR = 7, ORC_MAXNUM = 8, ORC_MINNUM = 9
};
enum { ORC_SKIP = 0, ORC_ZEROFILL = 1, ORC_CLAMP = 2 };
enum { ORC_IDX_I32 = 9, ORC_IDX_I64 = 10, ORC_IDX_U32 = 23 };

/* ---- codecs ------------------------------------------------------------------------- */
uint16_t orc_f32_to_bf16_bits(float x);
double orc_bf16_to_f64(uint16_t b);
double orc_f16_to_f64(uint16_t h);
uint16_t orc_f32_to_f16_bits(float x);
float orc_f64_to_f32_odd(double f);
uint16_t orc_store_bf16(double v);
void orc_f32_to_bf16_array(const float* x, int64_t n, uint16_t* out);
void orc_f16_to_f64_array(const uint16_t* h, int64_t n, double* out);

/* ---- sub-byte ------------------------------------------------------------------------ */
int32_t orc_u4_load(const uint8_t* p, int64_t i);
int32_t orc_i4_load(const uint8_t* p, int64_t i);
void orc_sub4_store(uint8_t* p, int64_t i, int32_t v);

/* ---- reductions (serial lift order) --------------------------------------------------- */
void orc_reduce_rows_f32(const float* in, int64_t rows, int64_t cols, int op, float* out);
void orc_reduce_rows_f64(const double* in, int64_t rows, int64_t cols, int op, double* out);
void orc_reduce_rows_i32(const int32_t* in, int64_t rows, int64_t cols, int op, int32_t* out);
void orc_reduce_rows_i64(const int64_t* in, int64_t rows, int64_t cols, int op, int64_t* out);
/* The launched lift's documented order for one row of floats (Sum/Mean): thread t of `block`
 * folds elements t, t+block, ... in f64, then the tree; one rounding at the end. */
double orc_sum_launched_order(const double* xs, int64_t n, int64_t block, int mean);
/* The declared bound on a float Sum/Mean row result `got` (stored at f32 when f32 != 0). */
double orc_sum_bound(const double* xs, int64_t n, int mean, int f32, double got);
double orc_neumaier(const double* xs, int64_t n);

/* ---- scans (serial lift order) -------------------------------------------------------- */
void orc_scan_rows_f32(const float* in, int64_t rows, int64_t cols, int op, int exclusive, int reverse, float* out);
void orc_scan_rows_f64(const double* in, int64_t rows, int64_t cols, int op, int exclusive, int reverse, double* out);
void orc_scan_rows_i32(const int32_t* in, int64_t rows, int64_t cols, int op, int exclusive, int reverse, int32_t* out);
void orc_scan_rows_i64(const int64_t* in, int64_t rows, int64_t cols, int op, int exclusive, int reverse, int64_t* out);
/* The launched scan's three-phase order for one row of f32 Sum (chunk c = ceil(n/block)). */
void orc_scan_launched_order_f32(const float* in, int64_t n, int64_t block, int exclusive, int reverse, float* out);

/* ---- gather ------------------------------------------------------------------------- */
/* out[r, :] = table[clamp(ids[r]), :] (rows of row_bytes raw bytes) under the policy. */
void orc_gather_rows(const uint8_t* table, int64_t src_extent, int64_t row_bytes, const void* ids, int idx_kind,
                     int64_t n_rows, int policy, uint8_t* out);

/* ---- sub-byte dequant ----------------------------------------------------------------- */
/* The dequantizing GEMM of crates/unpopped/tests/support/dequant.rs:104-181:
   out[r][c] = sum_k (w[r][k] - zero[r][k/group]) * scale[r][k/group] * x[k][c], every operation an
   I32 that wraps; w packed 4-bit (I4 sign-extends, U4 zero-extends), x I32 (x_i32) or I8. */
void orc_dequant_gemm_i32(const uint8_t* w, int w_signed, const int32_t* zero, const int32_t* scale, const void* x,
                          int x_i32, int64_t rows, int64_t k, int64_t cols, int64_t group, int32_t* out);
void orc_dequant4_bf16(const uint8_t* q, int q_signed, const uint16_t* scale, const uint8_t* zero, int z_signed,
                       int64_t rows, int64_t cols, int64_t group, uint16_t* out);

/* ---- row reduction (Access::RowReduce) ------------------------------------------------- */
/* An expression as a postfix program over a stack of doubles: leaves push, operators pop their
 * operands and push the result.  `arg` is the leaf's index or the operator's code. */
enum {
  ORC_RX_INPUT = 1, ORC_RX_REDUCED, ORC_RX_CONST, ORC_RX_ADD, ORC_RX_SUB, ORC_RX_MUL, ORC_RX_DIV,
  ORC_RX_FMA, ORC_RX_SELECT, ORC_RX_UNARY, ORC_RX_BINARY
};
typedef struct orc_rx {
  int32_t op;
  int32_t arg;
  double c;
} orc_rx;
/* Evaluate a program in f64 (crates/unpopped/src/oracle/expr_eval.rs over scalar_ops.rs);
 * `f32` is the compute dtype's width for Sign and Step. */
double orc_rx_eval(const orc_rx* prog, int32_t len, const double* x, const double* red, int f32);
/* The lifted serial row reduction (kernel_lift/row_reduce.rs:31-231 as the kernel evaluator
 * runs it): per row, each stage folds round_T(pre) in f64 in ascending column order (Max/Min
 * with the NaN rule), finalises and rounds once to T; the epilogue is evaluated in f64 and
 * rounded once at the store.  `f64` picks T (F64, else F32); `ins` are n_inputs row-major
 * rows x cols arrays of T. */
void orc_row_reduce(const void* const* ins, int32_t n_inputs, int64_t rows, int64_t cols, int f64, int32_t n_stages,
                    const int32_t* ops, const orc_rx* const* pres, const int32_t* pre_lens, const orc_rx* epi,
                    int32_t epi_len, void* out);
/* The lifted serial scan with a pre-map and a fused post (lift_scan_opdef, kernel_lift.rs:504-619,
 * as the kernel evaluator runs it): the inputs (n_inputs arrays of T, one shape) seen as A x S x B
 * around the scanned axis; at each position the pre is evaluated in f64 over the position's inputs
 * and rounded once to T, the fold takes it in f64 (fold_f64), the prefix is rounded once to T (a
 * running Mean divided by the count folded so far), and a post (post_len > 0) is evaluated in f64
 * over that prefix (Reduced(0)) and the position's inputs, rounded once at the store. */
void orc_scan_x(const void* const* ins, int32_t n_inputs, int64_t a_ext, int64_t s_ext, int64_t b_ext, int f64, int op,
                int exclusive, int reverse, const orc_rx* pre, int32_t pre_len, const orc_rx* post, int32_t post_len,
                void* out);

/* ---- Access::Elementwise (kernel_lift.rs:96-153 as the kernel evaluator runs it) ---------- */

/* out[i] = round_T(program(x_0[i], ..., x_{n-1}[i])) for i < count: the body evaluated in f64 and
 * rounded once at the store (the statement model, oracle/kernel_eval.rs:763-771; launch_cases.rs
 * :14-27).  `ins` are n_inputs arrays of T already in the output's element order; `f64` picks T. */
void orc_elementwise_f(const void* const* ins, int32_t n_inputs, int64_t count, int f64, const orc_rx* prog,
                       int32_t len, void* out);

/* An integer expression program (postfix): every node carries the integer kind it is evaluated
 * at (ORC_K_*), as eval_int (oracle/kernel_eval.rs:809-848) passes the type down: an operand at the
 * node's type, except a Cast's operand, a comparison's operands and a Select's condition, which
 * the program compiler types by the operand's own type. */
enum { ORC_K_I32 = 9, ORC_K_I64 = 10, ORC_K_U32 = 23, ORC_K_U64 = 24 };
enum {
  ORC_IX_INPUT = 1, ORC_IX_CONST, ORC_IX_CAST, ORC_IX_ADD, ORC_IX_SUB, ORC_IX_MUL, ORC_IX_DIV, ORC_IX_SHL,
  ORC_IX_SHR, ORC_IX_MIN, ORC_IX_MAX, ORC_IX_AND, ORC_IX_OR, ORC_IX_XOR, ORC_IX_CMP, ORC_IX_SELECT
};
typedef struct orc_ix {
  int32_t op;
  int32_t arg;  /* INPUT: the input; CMP: 0 Eq, 1 Ne, 2 Lt, 3 Le, 4 Gt, 5 Ge */
  int32_t kind; /* the kind the node's value is computed at */
  int32_t pad;
  int64_t v;    /* CONST: the literal */
} orc_ix;
/* Planted mistakes (tests only; 0 in every parity use): a zero divisor gives 0, MIN / -1
 * saturates to MAX, a shift count at or past the width clamps (as PTX does) instead of wrapping,
 * Shr is logical on a signed type, Div floors. */
enum { ORC_MUT_DIV0 = 1, ORC_MUT_MINNEG1 = 2, ORC_MUT_CLAMP = 4, ORC_MUT_LOGICAL = 8, ORC_MUT_FLOOR = 16 };
/* out[i] = program over the inputs' element i, each input an int64 array holding the compute
 * kind's value (a U64 value as its bit pattern); the result is stored as the kind's value the same
 * way. */
void orc_elementwise_i(const int64_t* const* ins, int32_t n_inputs, int64_t count, const orc_ix* prog, int32_t len,
                       int32_t mutant, int64_t* out);

#endif
