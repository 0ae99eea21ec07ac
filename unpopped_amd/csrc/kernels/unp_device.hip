// unpopped-hip device template library (gfx950, wave64).
//
// The HIP emitter writes a kernel source as: this library + one `extern "C" __global__`
// entry that instantiates one template below with the form's element type, fold, launch
// geometry and policy.  The Compiler turns that text into a code object (hipRTC); the
// runtime loads it with hipModuleLoadData and launches it with hipModuleLaunchKernel.
//
// Numerics follow the reference's lifts:
//   * float Sum / Mean fold in f64 and round once to the element type at the store
//     (crates/unpopped/src/kernel_lift.rs:883-896, :965-983);
//   * Max / Min keep a NaN once seen: `!have || v != v || better(v, acc)`
//     (kernel_lift.rs:1097-1160); the `have` flag is replaced by the monoid identity
//     (-inf / +inf / INT_MIN / INT_MAX), which the NaN-keeping step leaves unchanged;
//   * integer folds wrap at the element width (kernel_lift.rs:883-889);
//   * an empty fold stores the fold's starting value: 0 for Sum/Max/Min, 1 for Prod,
//     0/0 for Mean (kernel_lift.rs:915-924, :941-963);
//   * bf16 stores round to nearest even, a NaN keeps its top bits and is quieted
//     (crates/unpopped/src/oracle/float_codec.rs:259-266).
// The reduction order inside a kernel is fixed by the launch geometry, as the launched
// lifts fix theirs by (grid, block) (kernel_lift/block_reduce.rs:14-24); a float Sum is held
// to the declared bound gamma_(n-1) * sum|x| + half an ulp of the final rounding.
//
// Cross-lane work uses DPP (row_shr, wave_shr) and v_readlane; cross-wave work goes
// through LDS.  Global loads and stores are 128-bit where the host has checked the
// alignment (the `VEC` / `UNIT` template arguments).

#if !defined(__HIPCC_RTC__)
#include <hip/hip_runtime.h>
#endif

namespace unp {

typedef unsigned char u8;
typedef unsigned short u16;
typedef unsigned int u32;
typedef unsigned long long u64;
typedef int i32;
typedef long long i64;

#define UNP_DEV __device__ __forceinline__

enum : int {
  OP_SUM = 0, OP_PROD = 1, OP_MAX = 2, OP_MIN = 3, OP_MEAN = 4,
  OP_AND = 5, OP_OR = 6, OP_XOR = 7, OP_MAXNUM = 8, OP_MINNUM = 9
};
enum : int { OOB_SKIP = 0, OOB_ZEROFILL = 1, OOB_CLAMP = 2 };

template <class T> struct traits;
template <> struct traits<float> {
  static constexpr bool is_float = true;
  typedef u32 uns;
};
template <> struct traits<double> {
  static constexpr bool is_float = true;
  typedef u64 uns;
};
template <> struct traits<i32> {
  static constexpr bool is_float = false;
  typedef u32 uns;
  static constexpr i32 lo = -2147483647 - 1;
  static constexpr i32 hi = 2147483647;
};
template <> struct traits<i64> {
  static constexpr bool is_float = false;
  typedef u64 uns;
  static constexpr i64 lo = -9223372036854775807LL - 1;
  static constexpr i64 hi = 9223372036854775807LL;
};

// The accumulator: a float Sum or Mean folds in f64, every other fold at the element type
// (exact for Max/Min; wrapping for the integers).
template <class T, int OP> struct acc { typedef T type; };
template <> struct acc<float, OP_SUM> { typedef double type; };
template <> struct acc<float, OP_MEAN> { typedef double type; };

template <class A, int OP> struct fold;

template <class A> struct fold_sum {
  static UNP_DEV A identity() { return A(0); }
  static UNP_DEV A apply(A a, A b) {
    if constexpr (traits<A>::is_float) {
      return a + b;
    } else {
      typedef typename traits<A>::uns U;
      return (A)((U)a + (U)b);
    }
  }
};
template <class A> struct fold<A, OP_SUM> : fold_sum<A> {};
template <class A> struct fold<A, OP_MEAN> : fold_sum<A> {};

template <class A> struct fold<A, OP_PROD> {
  static UNP_DEV A identity() { return A(1); }
  static UNP_DEV A apply(A a, A b) {
    if constexpr (traits<A>::is_float) {
      return a * b;
    } else {
      typedef typename traits<A>::uns U;
      return (A)((U)a * (U)b);
    }
  }
};

template <class A> struct fold<A, OP_MAX> {
  static UNP_DEV A identity() {
    if constexpr (traits<A>::is_float) return A(-__builtin_inf());
    else return traits<A>::lo;
  }
  // `a` is the earlier partial; a NaN on either side is kept once seen.
  static UNP_DEV A apply(A a, A b) {
    if constexpr (traits<A>::is_float) return (b > a || b != b) ? b : a;
    else return b > a ? b : a;
  }
};

template <class A> struct fold<A, OP_MIN> {
  static UNP_DEV A identity() {
    if constexpr (traits<A>::is_float) return A(__builtin_inf());
    else return traits<A>::hi;
  }
  static UNP_DEV A apply(A a, A b) {
    if constexpr (traits<A>::is_float) return (b < a || b != b) ? b : a;
    else return b < a ? b : a;
  }
};

// MaxNum / MinNum ignore NaN: the quiet NaN is their identity (any value replaces it), so a run
// of only NaN folds to NaN.  On integers they are Max / Min.
template <class A> struct fold<A, OP_MAXNUM> {
  static UNP_DEV A identity() {
    if constexpr (traits<A>::is_float) return A(__builtin_nan(""));
    else return traits<A>::lo;
  }
  static UNP_DEV A apply(A a, A b) {
    if constexpr (traits<A>::is_float) return a != a ? b : ((b == b && b > a) ? b : a);
    else return b > a ? b : a;
  }
};
template <class A> struct fold<A, OP_MINNUM> {
  static UNP_DEV A identity() {
    if constexpr (traits<A>::is_float) return A(__builtin_nan(""));
    else return traits<A>::hi;
  }
  static UNP_DEV A apply(A a, A b) {
    if constexpr (traits<A>::is_float) return a != a ? b : ((b == b && b < a) ? b : a);
    else return b < a ? b : a;
  }
};

// Bitwise folds of the integers (associative and commutative: every order gives the same bits).
template <class A> struct fold<A, OP_AND> {
  static UNP_DEV A identity() { return (A)~(typename traits<A>::uns)0; }
  static UNP_DEV A apply(A a, A b) { return a & b; }
};
template <class A> struct fold<A, OP_OR> {
  static UNP_DEV A identity() { return A(0); }
  static UNP_DEV A apply(A a, A b) { return a | b; }
};
template <class A> struct fold<A, OP_XOR> {
  static UNP_DEV A identity() { return A(0); }
  static UNP_DEV A apply(A a, A b) { return a ^ b; }
};

// The value stored for a finished fold over `n` elements: an empty fold stores the lift's
// starting value 0 (kernel_lift.rs:899-906), whatever the fold's identity.
template <class T, int OP, class A> UNP_DEV T finish(A a, i64 n) {
  if constexpr (OP == OP_MEAN) {
    return (T)(a / (double)n);
  } else if constexpr (OP == OP_MAX || OP == OP_MIN || OP == OP_MAXNUM || OP == OP_MINNUM || OP == OP_AND) {
    return n == 0 ? T(0) : (T)a;
  } else {
    return (T)a;
  }
}

// ---------------------------------------------------------------------------------------
// Vectors and lane primitives
// ---------------------------------------------------------------------------------------

template <class T, int N> struct alignas(sizeof(T) * N) vec {
  T e[N];
};

template <class T, int N> UNP_DEV vec<T, N> ld(const T* p) {
  return *reinterpret_cast<const vec<T, N>*>(p);
}
template <class T, int N> UNP_DEV void stv(T* p, const vec<T, N>& v) {
  *reinterpret_cast<vec<T, N>*>(p) = v;
}

// Streaming (nontemporal) 16/8/4-byte vector accesses: data read or written once are not
// kept in the caches.  Other widths fall back to plain accesses.
typedef u32 u32x4_t __attribute__((ext_vector_type(4)));
typedef u32 u32x2_t __attribute__((ext_vector_type(2)));

template <class T, int N> UNP_DEV vec<T, N> ld_nt(const T* p) {
  if constexpr (sizeof(T) * N == 16) {
    return __builtin_bit_cast(vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
  } else if constexpr (sizeof(T) * N == 8) {
    return __builtin_bit_cast(vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p)));
  } else if constexpr (sizeof(T) * N == 4) {
    return __builtin_bit_cast(vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const u32*>(p)));
  } else {
    return ld<T, N>(p);
  }
}
template <class T, int N> UNP_DEV void st_nt(T* p, const vec<T, N>& v) {
  if constexpr (sizeof(T) * N == 16) {
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), reinterpret_cast<u32x4_t*>(p));
  } else if constexpr (sizeof(T) * N == 8) {
    __builtin_nontemporal_store(__builtin_bit_cast(u32x2_t, v), reinterpret_cast<u32x2_t*>(p));
  } else if constexpr (sizeof(T) * N == 4) {
    __builtin_nontemporal_store(__builtin_bit_cast(u32, v), reinterpret_cast<u32*>(p));
  } else {
    stv<T, N>(p, v);
  }
}

template <class X> UNP_DEV u64 to_bits64(X v) {
  if constexpr (sizeof(X) == 4) return (u64)__builtin_bit_cast(u32, v);
  else return __builtin_bit_cast(u64, v);
}
template <class X> UNP_DEV X from_bits64(u64 b) {
  if constexpr (sizeof(X) == 4) return __builtin_bit_cast(X, (u32)b);
  else return __builtin_bit_cast(X, b);
}

// v_mov_b32_dpp: lanes whose source is outside the row (or the wave) keep `old`.
template <int CTRL, int ROW_MASK> UNP_DEV u32 dpp32(u32 old, u32 src) {
  return (u32)__builtin_amdgcn_update_dpp((int)old, (int)src, CTRL, ROW_MASK, 0xF, false);
}

template <int CTRL, int ROW_MASK, class X> UNP_DEV X dpp(X old, X src) {
  if constexpr (sizeof(X) == 4) {
    return __builtin_bit_cast(
        X, dpp32<CTRL, ROW_MASK>(__builtin_bit_cast(u32, old), __builtin_bit_cast(u32, src)));
  } else {
    static_assert(sizeof(X) == 8, "4- or 8-byte lanes");
    const u64 o = __builtin_bit_cast(u64, old), s = __builtin_bit_cast(u64, src);
    const u32 lo = dpp32<CTRL, ROW_MASK>((u32)o, (u32)s);
    const u32 hi = dpp32<CTRL, ROW_MASK>((u32)(o >> 32), (u32)(s >> 32));
    return __builtin_bit_cast(X, ((u64)hi << 32) | (u64)lo);
  }
}

template <class X> UNP_DEV X settle(X x);

// v_readlane of a 4- or 8-byte value.  An 8-byte value is settled first (settle, below): the
// readlane may follow the VALU op that produced it by fewer wait states than gfx950 needs.
template <class X> UNP_DEV X readlane(X v, int lane) {
  if constexpr (sizeof(X) == 4) {
    return __builtin_bit_cast(X, (u32)__builtin_amdgcn_readlane((int)__builtin_bit_cast(u32, v), lane));
  } else {
    const u64 b = __builtin_bit_cast(u64, settle(v));
    const u32 lo = (u32)__builtin_amdgcn_readlane((int)(u32)b, lane);
    const u32 hi = (u32)__builtin_amdgcn_readlane((int)(u32)(b >> 32), lane);
    return __builtin_bit_cast(X, ((u64)hi << 32) | (u64)lo);
  }
}

// DPP control words (GFX9 encoding).
enum : int {
  DPP_ROW_SHR1 = 0x111,
  DPP_ROW_SHR2 = 0x112,
  DPP_ROW_SHR4 = 0x114,
  DPP_ROW_SHR8 = 0x118,
  DPP_WAVE_SHR1 = 0x138,
};

// Inclusive scan inside each 16-lane row (Hillis-Steele over row_shr 1, 2, 4, 8; the
// earlier lane is the left operand).  Must be called with all 64 lanes active.
template <class A, int OP> UNP_DEV A row_inclusive_scan(A x) {
  typedef fold<A, OP> F;
  const A I = F::identity();
  x = F::apply(dpp<DPP_ROW_SHR1, 0xF>(I, x), x);
  x = F::apply(dpp<DPP_ROW_SHR2, 0xF>(I, x), x);
  x = F::apply(dpp<DPP_ROW_SHR4, 0xF>(I, x), x);
  x = F::apply(dpp<DPP_ROW_SHR8, 0xF>(I, x), x);
  return x;
}

// Wait states between an 8-byte VALU result and a v_readlane of it.  On gfx950 a v_readlane
// issued one wait state after a v_add_f64 (all the compiler puts there) has returned the
// register's value from before the add: a wave scan's row totals, read at lanes 15/31/47/63,
// then lacked the last DPP steps.  The asm takes and returns the value, so its nops sit after
// the value's producer and before every reader.  4-byte values are not affected.  readlane
// settles every 8-byte value it reads, so no caller depends on doing it first.
template <class X> UNP_DEV X settle(X x) {
  if constexpr (sizeof(X) == 8) asm volatile("s_nop 4" : "+v"(x));
  return x;
}

// The fold of all 64 lanes, the same value in every lane.
template <class A, int OP> UNP_DEV A wave_reduce(A x) {
  typedef fold<A, OP> F;
  x = settle(row_inclusive_scan<A, OP>(x));
  return F::apply(F::apply(F::apply(readlane(x, 15), readlane(x, 31)), readlane(x, 47)),
                  readlane(x, 63));
}

// Inclusive scan over the 64 lanes (lane order = fold order).  The result is settled, so a
// caller may read it with readlane at once.
template <class A, int OP> UNP_DEV A wave_inclusive_scan(A x, int lane) {
  typedef fold<A, OP> F;
  x = settle(row_inclusive_scan<A, OP>(x));
  const A r0 = readlane(x, 15);
  const A r01 = F::apply(r0, readlane(x, 31));
  const A r012 = F::apply(r01, readlane(x, 47));
  const int row = lane >> 4;
  const A pre = row == 1 ? r0 : (row == 2 ? r01 : r012);
  return settle(row == 0 ? x : F::apply(pre, x));
}

// Lane l receives lane l-1's value; lane 0 receives `fill`.
template <class A> UNP_DEV A wave_shr1(A x, A fill) { return dpp<DPP_WAVE_SHR1, 0xF>(fill, x); }

// Fold of a value held by every thread of a block, in wave order; the same result in every
// thread.  `s` has one slot per wave.
template <class A, int OP, int THREADS> UNP_DEV A block_reduce(A x, A* s) {
  typedef fold<A, OP> F;
  constexpr int WAVES = THREADS / 64;
  x = wave_reduce<A, OP>(x);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = x;
  __syncthreads();
  A r = s[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) r = F::apply(r, s[w]);
  __syncthreads();
  return r;
}

// Arrive at a device-scope counter once this wave's stores have completed (vmcnt), so that the
// block drawing the last arrival usually finds every tagged partial already in place.  This
// only shortens the reader's wait: the reader checks each partial's tag itself (tagged<A>),
// and nothing here is needed for its correctness.  Returns the counter's previous value.
UNP_DEV u32 arrive_after_stores(u32* counter) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): expcnt and lgkmcnt left at their maximum
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Draw the next ticket of a device-scope counter (one lane).  An atomic increment, not an
// add: the compiler's atomic optimizer rewrites a one-lane add into a wave-aggregated form
// that waits for the returned value at once, where an increment's value is waited for only
// where it is used, so the draw's latency overlaps the loads issued after it.
UNP_DEV u32 draw_ticket(u32* counter) {
  return __builtin_amdgcn_atomic_inc32(counter, 0xffffffffu, __ATOMIC_RELAXED, "agent");
}

// ---------------------------------------------------------------------------------------
// Bounded waits.  A wave that waits for another block (a scan tile for its predecessors'
// status, a full reduction's folding block for the other blocks' partials, a staged scan's
// consumer waves for their tile's look-back) gives up once `ticks` of the device's constant
// wall clock (wall_clock64) have passed since its wait began, adds one to `*stall`, and goes
// on with the identity in place of what it waited for.  Every wave still reaches the end of
// the kernel, and the host reads the stall word to report the launch's outputs invalid instead
// of the device hanging on a lost predecessor.  With ticks = 0 a wait gives up at its first
// unanswered probe.
// ---------------------------------------------------------------------------------------
struct waits {
  u32* stall;
  u32 ticks;
};
static_assert(sizeof(waits) == 16, "the host passes a 16-byte waits argument");
UNP_DEV void note_stall(const waits& wt) {
  __hip_atomic_fetch_add(wt.stall, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// True once a wait that began at t0 has run out.
UNP_DEV bool wait_over(u64 t0, const waits& wt) { return wall_clock64() - t0 >= (u64)wt.ticks; }

// A value one block publishes for another, as W 64-bit words [launch epoch: 32 bits | 32 bits of
// the value].  The reader takes the value only when every word carries this launch's epoch, so
// the value arrives in the same atomic word as the tag that says it is complete: per-location
// coherence of the relaxed agent-scope accesses is all the hand-off relies on, and no ordering
// between different locations is needed (an agent-scope release / acquire pair would write back
// and invalidate the XCD's whole L2).  The host advances the epoch per launch and clears the
// words before the epoch wraps, so no reset is needed between launches.
// Word i of a value lies at p + i * stride: callers lay the words out in planes, so that the
// lanes of a wave store and load whole contiguous runs.
template <class A> struct tagged {
  static_assert(sizeof(A) == 4 || sizeof(A) == 8, "4- or 8-byte values");
  static constexpr int W = sizeof(A) == 4 ? 1 : 2;
  static UNP_DEV void put(u64* p, i64 stride, A v, u32 epoch) {
    const u64 b = to_bits64(v), tag = (u64)epoch << 32;
    __hip_atomic_store(p, tag | (b & 0xffffffffull), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (W == 2)
      __hip_atomic_store(p + stride, tag | (b >> 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  static UNP_DEV bool take(const u64* p, i64 stride, u32 epoch, A& v) {
    u64 w[W];
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = __hip_atomic_load(p + i * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool ok = (u32)(w[0] >> 32) == epoch;
    u64 b = w[0] & 0xffffffffull;
    if constexpr (W == 2) {
      ok = ok && (u32)(w[1] >> 32) == epoch;
      b |= w[1] << 32;
    }
    v = from_bits64<A>(b);
    return ok;
  }
  // The value at p, waiting for it (bounded); `ident` after a give-up.
  static UNP_DEV A wait(const u64* p, i64 stride, u32 epoch, A ident, const waits& wt) {
    A v;
    if (take(p, stride, epoch, v)) return v;
    const u64 t0 = wall_clock64();
    for (;;) {
      __builtin_amdgcn_s_sleep(1);
      if (take(p, stride, epoch, v)) return v;
      if (wait_over(t0, wt)) {
        note_stall(wt);
        return ident;
      }
    }
  }
};

// ---------------------------------------------------------------------------------------
// Row reduction, one wave per row: waves stride over rows (the outermost kept axis, as
// kernel_lift/block_reduce.rs:313-338 strides blocks over it); lane l folds the vectors
// l, l + 64, ... of its row (U of them in flight), then the wave combines by DPP and lane 0
// stores.  No LDS and no barrier: the schedule for rows up to a few thousand vectors.
// ---------------------------------------------------------------------------------------
template <class T, int OP0, int OP1, int NOUT, int VEC, int THREADS, int U>
UNP_DEV void rowreduce_wave(const T* __restrict__ in, T* __restrict__ out0, T* __restrict__ out1, i64 rows,
                            i64 cols) {
  typedef typename acc<T, OP0>::type A0;
  typedef typename acc<T, OP1>::type A1;
  typedef fold<A0, OP0> F0;
  typedef fold<A1, OP1> F1;
  constexpr i64 STEP = (i64)64 * VEC;
  const int lane = threadIdx.x & 63;
  const i64 nwaves = (i64)gridDim.x * (THREADS / 64);
  for (i64 row = (i64)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6); row < rows; row += nwaves) {
    const T* __restrict__ p = in + row * cols;
    A0 a0 = F0::identity();
    A1 a1 = F1::identity();
    i64 c = (i64)lane * VEC;
    for (; c + (U - 1) * STEP < cols; c += U * STEP) {
      vec<T, VEC> v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = ld_nt<T, VEC>(p + c + u * STEP);
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          a0 = F0::apply(a0, (A0)v[u].e[e]);
          if constexpr (NOUT > 1) a1 = F1::apply(a1, (A1)v[u].e[e]);
        }
      }
    }
    for (; c < cols; c += STEP) {
      const vec<T, VEC> v = ld_nt<T, VEC>(p + c);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        a0 = F0::apply(a0, (A0)v.e[e]);
        if constexpr (NOUT > 1) a1 = F1::apply(a1, (A1)v.e[e]);
      }
    }
    a0 = wave_reduce<A0, OP0>(a0);
    if constexpr (NOUT > 1) a1 = wave_reduce<A1, OP1>(a1);
    if (lane == 0) {
      out0[row] = finish<T, OP0>(a0, cols);
      if constexpr (NOUT > 1) out1[row] = finish<T, OP1>(a1, cols);
    }
  }
}

// ---------------------------------------------------------------------------------------
// Row reduction, one block per row: rows x cols row-major, one or two folds of each row read
// once.  Blocks stride over rows (row = blockIdx.x; += gridDim.x), as the launched reduction
// lift strides over its outermost kept axis (kernel_lift/block_reduce.rs:313-338).
// Inside a row, thread t folds the vectors t, t + THREADS, ... (VEC elements each) in
// ascending order; waves combine by DPP, blocks by LDS in wave order.
// ---------------------------------------------------------------------------------------
template <class T, int OP0, int OP1, int NOUT, int VEC, int THREADS, int UNROLL>
UNP_DEV void rowreduce(const T* __restrict__ in, T* __restrict__ out0, T* __restrict__ out1, i64 rows,
                       i64 cols) {
  typedef typename acc<T, OP0>::type A0;
  typedef typename acc<T, OP1>::type A1;
  typedef fold<A0, OP0> F0;
  typedef fold<A1, OP1> F1;
  constexpr int WAVES = THREADS / 64;
  constexpr i64 STEP = (i64)THREADS * VEC;
  __shared__ A0 s0[2][WAVES];
  __shared__ A1 s1[2][WAVES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int par = 0;
  for (i64 row = blockIdx.x; row < rows; row += gridDim.x) {
    const T* __restrict__ p = in + row * cols;
    A0 a0 = F0::identity();
    A1 a1 = F1::identity();
    i64 c = (i64)tid * VEC;
    for (; c + (UNROLL - 1) * STEP < cols; c += UNROLL * STEP) {
      vec<T, VEC> v[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) v[u] = ld_nt<T, VEC>(p + c + u * STEP);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          a0 = F0::apply(a0, (A0)v[u].e[e]);
          if constexpr (NOUT > 1) a1 = F1::apply(a1, (A1)v[u].e[e]);
        }
      }
    }
    for (; c < cols; c += STEP) {
      const vec<T, VEC> v = ld_nt<T, VEC>(p + c);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        a0 = F0::apply(a0, (A0)v.e[e]);
        if constexpr (NOUT > 1) a1 = F1::apply(a1, (A1)v.e[e]);
      }
    }
    a0 = wave_reduce<A0, OP0>(a0);
    if constexpr (NOUT > 1) a1 = wave_reduce<A1, OP1>(a1);
    if (lane == 0) {
      s0[par][wave] = a0;
      if constexpr (NOUT > 1) s1[par][wave] = a1;
    }
    __syncthreads();
    if (tid == 0) {
      A0 r0 = s0[par][0];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) r0 = F0::apply(r0, s0[par][w]);
      out0[row] = finish<T, OP0>(r0, cols);
      if constexpr (NOUT > 1) {
        A1 r1 = s1[par][0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) r1 = F1::apply(r1, s1[par][w]);
        out1[row] = finish<T, OP1>(r1, cols);
      }
    }
    // The next row writes the other half of the LDS slots; the row after that reuses these
    // only after every thread has passed the next row's barrier.
    par ^= 1;
  }
}

// ---------------------------------------------------------------------------------------
// Full reduction of n elements to one value (no kept axis), in one launch: every block
// folds a grid-strided slice, publishes its partial, and the block that draws the last
// ticket folds the partials in block order and stores.  The order depends on
// (gridDim.x, THREADS, VEC, UNROLL) only, so the result is reproducible run to run.
// `counter` is zero on entry and is left zero; the partials are tagged with the launch's `epoch`
// and the folding block waits for each (bounded by `wt`).
// ---------------------------------------------------------------------------------------
template <class T, int OP, int VEC, int THREADS, int UNROLL>
UNP_DEV void reduce_all(const T* __restrict__ in, T* __restrict__ out, i64 n, u64* __restrict__ partials,
                        u32* __restrict__ counter, u32 epoch, waits wt) {
  typedef typename acc<T, OP>::type A;
  typedef fold<A, OP> F;
  constexpr int WAVES = THREADS / 64;
  __shared__ A s[WAVES];
  __shared__ u32 last;
  const int tid = threadIdx.x;
  const i64 STEP = (i64)gridDim.x * THREADS * VEC;
  A a = F::identity();
  i64 c = ((i64)blockIdx.x * THREADS + tid) * VEC;
  for (; c + (UNROLL - 1) * STEP < n; c += UNROLL * STEP) {
    vec<T, VEC> v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = ld_nt<T, VEC>(in + c + u * STEP);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) a = F::apply(a, (A)v[u].e[e]);
    }
  }
  for (; c < n; c += STEP) {
    const vec<T, VEC> v = ld_nt<T, VEC>(in + c);
#pragma unroll
    for (int e = 0; e < VEC; ++e) a = F::apply(a, (A)v.e[e]);
  }
  a = block_reduce<A, OP, THREADS>(a, s);
  typedef tagged<A> P;
  if (tid == 0) {
    P::put(partials + blockIdx.x, gridDim.x, a, epoch);
    last = (arrive_after_stores(counter) == gridDim.x - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (last == 0u) return;
  A b = F::identity();
  for (u32 i = tid; i < gridDim.x; i += THREADS) b = F::apply(b, P::wait(partials + i, gridDim.x, epoch, F::identity(), wt));
  b = block_reduce<A, OP, THREADS>(b, s);
  if (tid == 0) {
    out[0] = finish<T, OP>(b, n);
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------------------
// Reduction of the middle axis of A x R x B (row-major): out[a, b] = fold_i in[a, i, b].  The
// shape every reduced-axis set with one contiguous run of reduced axes and kept axes after it
// takes once adjacent axes of a kind are merged (A = 1: the outer axis, as column sums).
//
// A wave covers 64 * VEC consecutive columns b of one a; the block's WAVES waves split the
// block's run of rows into WAVES consecutive pieces; the blocks of one column strip split R
// into S consecutive chunks.  The (strip, chunk) items are numbered chunk-major and blocks stride
// over them (a device-class grid), so consecutive blocks take consecutive strips of one chunk and
// the blocks in flight together read whole rows.  Lane l folds its VEC columns down its rows in ascending order
// (16-byte loads, every load of a wave instruction contiguous, U rows in flight); the waves
// meet in LDS in wave order; with S > 1 each block publishes its partials and the block that
// draws the strip's last ticket folds the S partials in chunk order and stores.  The order is
// fixed by (S, WAVES, U), so the result is reproducible.  counters[strip] is zero on entry and
// left zero; the chunk partials are tagged with the launch's `epoch` (tagged<A>).
// ---------------------------------------------------------------------------------------
template <class T, int OP, int VEC, int THREADS, int U>
UNP_DEV void reduce_mid(const T* __restrict__ in, T* __restrict__ out, i64 A, i64 R, i64 B, i64 S,
                        u64* __restrict__ partials, u32* __restrict__ counters, u32 epoch, waits wt) {
  typedef typename acc<T, OP>::type Ac;
  typedef fold<Ac, OP> F;
  constexpr int WAVES = THREADS / 64;
  typedef tagged<Ac> P;
  constexpr i64 CW = (i64)64 * VEC;  // columns per strip
  __shared__ Ac sh[WAVES][64 * VEC];
  __shared__ u32 last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const i64 ncb = (B + CW - 1) / CW;
  const i64 nstrips = A * ncb;
  // Items (strip, chunk), item = s * nstrips + strip; blocks stride over them.
  for (i64 item = blockIdx.x; item < nstrips * S; item += gridDim.x) {
    const i64 strip = item % nstrips;  // a * ncb + cb
    const i64 s = item / nstrips;
    const i64 a = strip / ncb, cb = strip - a * ncb;
    const i64 b0 = cb * CW + (i64)lane * VEC;
    const bool live = b0 < B;  // VEC divides B (the host picks VEC = 1 otherwise)
    // This item's rows [i0, i1), then this wave's piece of them.
    const i64 i0 = (R * s) / S, i1 = (R * (s + 1)) / S;
    const i64 w0 = i0 + ((i1 - i0) * wave) / WAVES, w1 = i0 + ((i1 - i0) * (wave + 1)) / WAVES;
    Ac acc_[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc_[e] = F::identity();
    if (live) {
      const T* __restrict__ p = in + (a * R) * B + b0;
      i64 i = w0;
      for (; i + U <= w1; i += U) {
        vec<T, VEC> v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = ld_nt<T, VEC>(p + (i + u) * B);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc_[e] = F::apply(acc_[e], (Ac)v[u].e[e]);
      }
      for (; i < w1; ++i) {
        const vec<T, VEC> v = ld_nt<T, VEC>(p + i * B);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc_[e] = F::apply(acc_[e], (Ac)v.e[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) sh[wave][lane * VEC + e] = acc_[e];
    __syncthreads();
    // Wave 0 folds the waves' partials in wave order.
    if (wave == 0) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        Ac r = sh[0][lane * VEC + e];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) r = F::apply(r, sh[w][lane * VEC + e]);
        acc_[e] = r;
      }
      if (S == 1) {
        if (live) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) out[a * B + b0 + e] = finish<T, OP>(acc_[e], R);
        }
      } else {
        // An item's partials: VEC x W planes of 64 words, word (e, i) of lane l at (e W + i) 64 + l.
        u64* __restrict__ mine = partials + (strip * S + s) * CW * P::W + lane;
#pragma unroll
        for (int e = 0; e < VEC; ++e) P::put(mine + e * P::W * 64, 64, acc_[e], epoch);
        if (lane == 0) last = (arrive_after_stores(&counters[strip]) == (u32)(S - 1)) ? 1u : 0u;
      }
    }
    if (S > 1) {
      __syncthreads();
      if (last != 0u && wave == 0) {
        // The strip's chunk partials, 8 chunks in flight at a time, each taken once its tag
        // shows this launch's epoch.
        Ac r[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) r[e] = F::identity();
        const u64* __restrict__ col = partials + strip * S * CW * P::W + lane;
        const i64 ITEM = CW * P::W;  // words from one chunk's partials to the next
        i64 k = 0;
        for (; k + 8 <= S; k += 8) {
          Ac v[8][VEC];
          bool ok = true;
#pragma unroll
          for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int e = 0; e < VEC; ++e) ok = P::take(col + (k + t) * ITEM + e * P::W * 64, 64, epoch, v[t][e]) && ok;
          if (!ok) {  // a partial not yet visible: wait for each in turn
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
              for (int e = 0; e < VEC; ++e)
                v[t][e] = P::wait(col + (k + t) * ITEM + e * P::W * 64, 64, epoch, F::identity(), wt);
          }
#pragma unroll
          for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int e = 0; e < VEC; ++e) r[e] = F::apply(r[e], v[t][e]);
        }
        for (; k < S; ++k)
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            r[e] = F::apply(r[e], P::wait(col + k * ITEM + e * P::W * 64, 64, epoch, F::identity(), wt));
        if (live) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) out[a * B + b0 + e] = finish<T, OP>(r[e], R);
        }
        if (lane == 0) __hip_atomic_store(&counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();  // sh and last are the next item's
  }
}

// ---------------------------------------------------------------------------------------
// Any reduced-axis set: one wave per output element.  The host passes the kept and the
// reduced axes (extents and element strides, outermost first, adjacent axes of a kind
// merged); output o unravels over the kept axes to its base offset, and lane l folds the
// reduced positions l, l + 64, ... (row-major over the reduced axes) before the wave's DPP
// combine.  Correct for every mask; the fast shapes above take the common ones.
// ---------------------------------------------------------------------------------------
struct axes_desc {
  i64 nk, nr;           // kept / reduced axis counts (after merging)
  i64 kext[8], kstr[8];
  i64 rext[8], rstr[8];
  i64 outs, count;      // output elements, reduced positions per output
};

template <class T, int OP, int THREADS>
UNP_DEV void reduce_generic(const T* __restrict__ in, T* __restrict__ out, const axes_desc& d) {
  typedef typename acc<T, OP>::type Ac;
  typedef fold<Ac, OP> F;
  const int lane = threadIdx.x & 63;
  const i64 nw = (i64)gridDim.x * (THREADS / 64);
  for (i64 o = (i64)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6); o < d.outs; o += nw) {
    i64 base = 0, q = o;
    for (i64 k = d.nk - 1; k >= 0; --k) {
      const i64 c = q % d.kext[k];
      q /= d.kext[k];
      base += c * d.kstr[k];
    }
    Ac a = F::identity();
    for (i64 t = lane; t < d.count; t += 64) {
      i64 off = base, u = t;
      for (i64 k = d.nr - 1; k >= 0; --k) {
        const i64 c = u % d.rext[k];
        u /= d.rext[k];
        off += c * d.rstr[k];
      }
      a = F::apply(a, (Ac)in[off]);
    }
    a = wave_reduce<Ac, OP>(a);
    if (lane == 0) out[o] = finish<T, OP>(a, d.count);
  }
}

// A reduction over storage images (oracle/buffers.rs:16-42): the kept axes with their input and
// output element strides, the reduced axes with their input strides, any signs.  A dense
// row-major reduction is the special case of row-major strides.
struct red_view {
  i64 nk, nr;
  i64 kext[8], kstr[8], kost[8];
  i64 rext[8], rstr[8];
  i64 outs, count;
};

// The serial lifts' accumulator: f64 for every float op (kernel_lift.rs:883-896), the dtype
// itself for an integer.
template <class T> struct serial_acc { typedef T type; };
template <> struct serial_acc<float> { typedef double type; };

// ---------------------------------------------------------------------------------------
// The serial lift's own order (kernel_lift.rs:447-484, reduce_loop :919-941): one lane per
// output, the reduced positions ascending in row-major order over the reduced axes folded into
// the serial accumulator (f64 for a float, the dtype itself for an integer), one rounding at the
// store.  The fold functors applied from their identity in this order make exactly the serial
// lift's steps (the `have` flag's first assignment included: kernel_lift.rs:1097-1160), so this is
// bit-exact to the serial kernel for every op, NaN payloads and signed zeros included.  The
// schedule of a float Prod (every product rounds; no declared bound) and the serial schedule of
// every reduction; not fast (each lane's fold is a dependent chain).
// ---------------------------------------------------------------------------------------
template <class T, int OP, int THREADS>
UNP_DEV void reduce_serial(const T* __restrict__ in, T* __restrict__ out, const red_view d) {
  typedef typename serial_acc<T>::type Ac;
  typedef fold<Ac, OP> F;
  const i64 stride = (i64)gridDim.x * THREADS;
  for (i64 o = (i64)blockIdx.x * THREADS + threadIdx.x; o < d.outs; o += stride) {
    i64 off = 0, oo = 0, q = o;
    for (i64 k = d.nk - 1; k >= 0; --k) {
      const i64 c = q % d.kext[k];
      q /= d.kext[k];
      off += c * d.kstr[k];
      oo += c * d.kost[k];
    }
    i64 ctr[8];
    for (i64 k = 0; k < d.nr; ++k) ctr[k] = 0;
    Ac a = F::identity();
    for (i64 t = 0; t < d.count; ++t) {
      a = F::apply(a, (Ac)in[off]);
      // Advance the odometer over the reduced axes (innermost fastest).
      for (i64 k = d.nr - 1; k >= 0; --k) {
        off += d.rstr[k];
        if (++ctr[k] < d.rext[k]) break;
        off -= d.rext[k] * d.rstr[k];
        ctr[k] = 0;
      }
    }
    out[oo] = finish<T, OP>(a, d.count);
  }
}

// Any order-free fold over storage images: one wave per output (as reduce_generic), the input and
// the output read and written through their strides.
template <class T, int OP, int THREADS>
UNP_DEV void reduce_strided(const T* __restrict__ in, T* __restrict__ out, const red_view d) {
  typedef typename acc<T, OP>::type Ac;
  typedef fold<Ac, OP> F;
  const int lane = threadIdx.x & 63;
  const i64 nw = (i64)gridDim.x * (THREADS / 64);
  for (i64 o = (i64)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6); o < d.outs; o += nw) {
    i64 base = 0, oo = 0, q = o;
    for (i64 k = d.nk - 1; k >= 0; --k) {
      const i64 c = q % d.kext[k];
      q /= d.kext[k];
      base += c * d.kstr[k];
      oo += c * d.kost[k];
    }
    Ac a = F::identity();
    for (i64 t = lane; t < d.count; t += 64) {
      i64 off = base, u = t;
      for (i64 k = d.nr - 1; k >= 0; --k) {
        const i64 c = u % d.rext[k];
        u /= d.rext[k];
        off += c * d.rstr[k];
      }
      a = F::apply(a, (Ac)in[off]);
    }
    a = wave_reduce<Ac, OP>(a);
    if (lane == 0) out[oo] = finish<T, OP>(a, d.count);
  }
}

// ---------------------------------------------------------------------------------------
// Reductions with a pre-map body over NI inputs and a fused post (the reduction lift with a
// non-plain body or post: kernel_lift.rs:919-941, 987-1003).  Float compute dtypes: at each
// position the body is evaluated in f64 over the inputs and rounded once to T, the fold runs in
// f64, the finished fold (Mean divided) is rounded once to T, and the post is evaluated in f64
// over that value and rounded once at the store.  Integer compute dtypes (I32, I64; no post,
// kernel_lift.rs:763-800): the body is evaluated at T by the total integer rule and the fold
// wraps at T, so every order gives the serial kernel's bits.  The emitted source supplies OPS:
// `arg` (the type the body reads its inputs at), `acc` (the fold's), `pre(x)` over the NI input
// values, `post(r)` over r[0], and `has_post`.
// ---------------------------------------------------------------------------------------
template <class T, int OP, class OPS, class Ac> UNP_DEV T xfinish(Ac a, i64 n) {
  const T red = finish<T, OP>(a, n);
  if constexpr (OPS::has_post) {
    const double r[1] = {(double)red};
    return (T)OPS::post(r);
  } else {
    return red;
  }
}

// The trailing run: rows x cols, one wave per row (U vectors of each input in flight per lane).
template <class T, int NI, int OP, class OPS, int VEC, int THREADS, int U>
UNP_DEV void xreduce_rows(const T* const* __restrict__ in, T* __restrict__ out, i64 rows, i64 cols) {
  typedef typename OPS::acc Ac;
  typedef typename OPS::arg X;
  typedef fold<Ac, OP> F;
  constexpr i64 STEP = (i64)64 * VEC;
  const int lane = threadIdx.x & 63;
  const i64 nwaves = (i64)gridDim.x * (THREADS / 64);
  for (i64 row = (i64)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6); row < rows; row += nwaves) {
    Ac a = F::identity();
    auto take = [&](const vec<T, VEC> (&v)[NI]) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        X x[NI];
#pragma unroll
        for (int k = 0; k < NI; ++k) x[k] = (X)v[k].e[e];
        a = F::apply(a, (Ac)(T)OPS::pre(x));
      }
    };
    i64 c = (i64)lane * VEC;
    for (; c + (U - 1) * STEP < cols; c += U * STEP) {
      vec<T, VEC> v[U][NI];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < NI; ++k) v[u][k] = ld_nt<T, VEC>(in[k] + row * cols + c + u * STEP);
#pragma unroll
      for (int u = 0; u < U; ++u) take(v[u]);
    }
    for (; c < cols; c += STEP) {
      vec<T, VEC> v[NI];
#pragma unroll
      for (int k = 0; k < NI; ++k) v[k] = ld_nt<T, VEC>(in[k] + row * cols + c);
      take(v);
    }
    a = wave_reduce<Ac, OP>(a);
    if (lane == 0) out[row] = xfinish<T, OP, OPS>(a, cols);
  }
}

// No kept axis: blocks fold grid-strided slices, the last block to arrive folds the partials
// in block order (the full reduction's protocol; `counter` zero on entry, left zero).
template <class T, int NI, int OP, class OPS, int VEC, int THREADS, int UNROLL>
UNP_DEV void xreduce_all(const T* const* __restrict__ in, T* __restrict__ out, i64 n, u64* __restrict__ partials,
                         u32* __restrict__ counter, u32 epoch, waits wt) {
  typedef typename OPS::acc Ac;
  typedef typename OPS::arg X;
  typedef fold<Ac, OP> F;
  constexpr int WAVES = THREADS / 64;
  __shared__ Ac sh[WAVES];
  __shared__ u32 last;
  const int tid = threadIdx.x;
  const i64 STEP = (i64)gridDim.x * THREADS * VEC;
  Ac a = F::identity();
  auto take = [&](const vec<T, VEC> (&v)[NI]) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      X x[NI];
#pragma unroll
      for (int k = 0; k < NI; ++k) x[k] = (X)v[k].e[e];
      a = F::apply(a, (Ac)(T)OPS::pre(x));
    }
  };
  i64 c = ((i64)blockIdx.x * THREADS + tid) * VEC;
  for (; c + (UNROLL - 1) * STEP < n; c += UNROLL * STEP) {
    vec<T, VEC> v[UNROLL][NI];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int k = 0; k < NI; ++k) v[u][k] = ld_nt<T, VEC>(in[k] + c + u * STEP);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) take(v[u]);
  }
  for (; c < n; c += STEP) {
    vec<T, VEC> v[NI];
#pragma unroll
    for (int k = 0; k < NI; ++k) v[k] = ld_nt<T, VEC>(in[k] + c);
    take(v);
  }
  a = block_reduce<Ac, OP, THREADS>(a, sh);
  typedef tagged<Ac> P;
  if (tid == 0) {
    P::put(partials + blockIdx.x, gridDim.x, a, epoch);
    last = (arrive_after_stores(counter) == gridDim.x - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (last == 0u) return;
  Ac b = F::identity();
  for (u32 i = tid; i < gridDim.x; i += THREADS)
    b = F::apply(b, P::wait(partials + i, gridDim.x, epoch, F::identity(), wt));
  b = block_reduce<Ac, OP, THREADS>(b, sh);
  if (tid == 0) {
    out[0] = xfinish<T, OP, OPS>(b, n);
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Any other reduced-axis set: one wave per output element (as reduce_generic), NI inputs of one
// shape read at the same offsets.
template <class T, int NI, int OP, class OPS, int THREADS>
UNP_DEV void xreduce_generic(const T* const* __restrict__ in, T* __restrict__ out, const axes_desc& d) {
  typedef typename OPS::acc Ac;
  typedef typename OPS::arg X;
  typedef fold<Ac, OP> F;
  const int lane = threadIdx.x & 63;
  const i64 nw = (i64)gridDim.x * (THREADS / 64);
  for (i64 o = (i64)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6); o < d.outs; o += nw) {
    i64 base = 0, q = o;
    for (i64 k = d.nk - 1; k >= 0; --k) {
      const i64 c = q % d.kext[k];
      q /= d.kext[k];
      base += c * d.kstr[k];
    }
    Ac a = F::identity();
    for (i64 t = lane; t < d.count; t += 64) {
      i64 off = base, u = t;
      for (i64 k = d.nr - 1; k >= 0; --k) {
        const i64 c = u % d.rext[k];
        u /= d.rext[k];
        off += c * d.rstr[k];
      }
      X x[NI];
#pragma unroll
      for (int k = 0; k < NI; ++k) x[k] = (X)in[k][off];
      a = F::apply(a, (Ac)(T)OPS::pre(x));
    }
    a = wave_reduce<Ac, OP>(a);
    if (lane == 0) out[o] = xfinish<T, OP, OPS>(a, d.count);
  }
}

// A scan's stored prefix: the fold rounded once to T, or for a running Mean the f64 sum divided by
// the count folded so far (scan_stored, kernel_lift.rs:604-619; an exclusive first prefix is 0 / 0).
template <class T, int OP, class A> UNP_DEV T scan_out(A v, i64 count) {
  if constexpr (OP == OP_MEAN) return (T)(v / (double)count);
  else return (T)v;
}


// ---------------------------------------------------------------------------------------
// A scan in the serial lift's own order (lift_scan_opdef, kernel_lift.rs:504-700): along a
// non-innermost axis of A x S x B, or a float Prod (every product rounds; no declared bound).
// One lane per column (a, b), lanes of a wave on consecutive b so that a wave's loads and stores
// of one step are contiguous; the scanned axis walked ascending (descending for a reverse scan),
// the prefix folded in the serial accumulator, a Mean divided by the count so far, each prefix
// rounded once at its store.  Bit-exact to the serial lift for every op and dtype.  U loads of a
// column are issued before its U stores, so one wait covers them.
// ---------------------------------------------------------------------------------------
template <class T, int OP, bool EXCL, bool REV, int U>
UNP_DEV void scan_seq(const T* __restrict__ in, T* __restrict__ out, i64 A, i64 S, i64 B) {
  typedef typename serial_acc<T>::type Ac;
  typedef fold<Ac, OP> F;
  const i64 cols = A * B;
  const i64 stride = (i64)gridDim.x * blockDim.x;
  for (i64 c = (i64)blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += stride) {
    const i64 a = c / B, b = c - a * B;
    const i64 base = a * S * B + b;
    Ac v = F::identity();
    i64 i = 0;
    for (; i + U <= S; i += U) {
      T x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) x[u] = in[base + (REV ? S - 1 - (i + u) : i + u) * B];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const i64 off = base + (REV ? S - 1 - (i + u) : i + u) * B;
        if constexpr (EXCL) {
          out[off] = scan_out<T, OP>(v, i + u);
          v = F::apply(v, (Ac)x[u]);
        } else {
          v = F::apply(v, (Ac)x[u]);
          out[off] = scan_out<T, OP>(v, i + u + 1);
        }
      }
    }
    for (; i < S; ++i) {
      const i64 off = base + (REV ? S - 1 - i : i) * B;
      const T xv = in[off];
      if constexpr (EXCL) {
        out[off] = scan_out<T, OP>(v, i);
        v = F::apply(v, (Ac)xv);
      } else {
        v = F::apply(v, (Ac)xv);
        out[off] = scan_out<T, OP>(v, i + 1);
      }
    }
  }
}

// A scan over storage images: the non-scanned axes (extents, input and output strides) and the
// scanned axis (extent, input and output strides), any signs.  One lane per column, the serial
// lift's order (as scan_seq): bit-exact for every op.
struct scan_view {
  i64 nc;
  i64 cext[8], cin[8], cout[8];
  i64 S, sin, sout;
  i64 cols;
};

template <class T, int OP, bool EXCL, bool REV>
UNP_DEV void scan_strided(const T* __restrict__ in, T* __restrict__ out, const scan_view v) {
  typedef typename serial_acc<T>::type Ac;
  typedef fold<Ac, OP> F;
  const i64 stride = (i64)gridDim.x * blockDim.x;
  for (i64 c = (i64)blockIdx.x * blockDim.x + threadIdx.x; c < v.cols; c += stride) {
    i64 bi = 0, bo = 0, q = c;
    for (i64 k = v.nc - 1; k >= 0; --k) {
      const i64 x = q % v.cext[k];
      q /= v.cext[k];
      bi += x * v.cin[k];
      bo += x * v.cout[k];
    }
    Ac acc_ = F::identity();
    for (i64 i = 0; i < v.S; ++i) {
      const i64 s = REV ? v.S - 1 - i : i;
      const T x = in[bi + s * v.sin];
      T* o = out + bo + s * v.sout;
      if constexpr (EXCL) {
        *o = scan_out<T, OP>(acc_, i);
        acc_ = F::apply(acc_, (Ac)x);
      } else {
        acc_ = F::apply(acc_, (Ac)x);
        *o = scan_out<T, OP>(acc_, i + 1);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Single-pass scan with decoupled look-back, along the innermost axis of rows x cols.
//
// A block tile is BT = WPB * 64 * VEC * K consecutive scan positions of one row.  Blocks are
// persistent: each round, one thread draws a tile ticket from `counter` (the next round's
// ticket is drawn at the start of the current round, so its latency overlaps the work).  A
// block only ever waits on tiles of lower index, whose tickets were drawn earlier by running
// blocks, so every wait ends.  Inside the tile wave w owns positions w * 64 * VEC * K ..:
// load k of lane l covers (k * 64 + l) * VEC .. + VEC of them, so every load instruction
// reads 64 * VEC contiguous elements, streamed past the caches.  The scan across a stripe is
// DPP; the waves' aggregates meet in LDS; one look-back per block tile (64 tiles per probe).
//
// Tile status: per tile W 64-bit words (W = 1 for a 4-byte carry, 2 for an 8-byte one), each
// [launch epoch: 31 bits | inclusive flag: 1 bit | 32 bits of the value].  A tile publishes
// its aggregate (flag 0) and later overwrites it with its inclusive prefix (flag 1).  A reader
// takes the words only when every one carries this launch's epoch and the same flag (a W = 2
// reader that catches the overwrite half done sees mixed flags and reads again), so one load
// per word answers a probe, and no fence and no reset is needed between launches.  The host
// advances `epoch` (1 .. 2^31 - 1) and `ticket_base` per launch.
// ---------------------------------------------------------------------------------------
template <class A, int SP = 0> struct tile_status {
  static constexpr int W = sizeof(A) == 4 ? 1 : 2;
  // Words from one tile's status to the next: W packs them densely; a wider stride spreads
  // the status of consecutive tiles, which every block probes at once, over cache lines and
  // memory channels.
  static constexpr int STRIDE = SP > W ? SP : W;

  // slot 0: the aggregate, slot 1: the inclusive prefix.
  static UNP_DEV void publish(u64* st, u64 tile, int slot, A v, u32 epoch) {
    u64* p = st + tile * STRIDE;
    const u64 b = to_bits64(v);
    const u64 tag = ((u64)epoch << 33) | ((u64)(slot == 1) << 32);
    __hip_atomic_store(p, tag | (b & 0xffffffffull), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (W == 2) {
      __hip_atomic_store(p + 1, tag | (b >> 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // Load a tile's words (all in flight together: one round trip).
  static UNP_DEV void fetch(const u64* st, u64 tile, u64 (&w)[W]) {
    const u64* p = st + tile * STRIDE;
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // 2: inclusive prefix in `v`; 1: aggregate in `v`; 0: nothing usable yet.
  static UNP_DEV int decode(const u64 (&w)[W], u32 epoch, A& v) {
    const u64 inc = (w[0] >> 32) & 1;
    bool ok = (w[0] >> 33) == (u64)epoch;
    u64 b = w[0] & 0xffffffffull;
    if constexpr (W == 2) {
      ok = ok && (w[1] >> 33) == (u64)epoch && ((w[1] >> 32) & 1) == inc;
      b |= w[1] << 32;
    }
    v = from_bits64<A>(b);
    return ok ? (inc ? 2 : 1) : 0;
  }
  static UNP_DEV int probe(const u64* st, u64 tile, u32 epoch, A& v) {
    u64 w[W];
    fetch(st, tile, w);
    return decode(w, epoch, v);
  }
};

// The fold of every earlier tile of this row (j = tile's index in its row, j >= 1).
// Lane l inspects the tiles l + 1, l + 65, ... back, P windows of 64 per round trip (the
// probes of all P are in flight together); the walk stops at the first inclusive prefix.
// A lane whose tile stays unpublished past the wait bound takes it as an inclusive identity,
// which ends the walk (the stall is counted; the result is then not the prefix).
//
// The walk is split in two: lookback_issue loads the first P windows' words and returns at
// once; lookback_finish decodes them and walks on.  A caller that has other work puts it
// between the two, so the first round trip overlaps it; lookback does both back to back.
// Lanes before the row's first tile read the current tile's own words (a valid address) and
// take the identity.
template <class A, int P, int SP>
UNP_DEV void lookback_issue(const u64* st, u64 tile, i64 j, int lane,
                            u64 (&w)[P][tile_status<A, SP>::W]) {
  typedef tile_status<A, SP> S;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const i64 pj = j - 1 - lane - 64 * p;
    S::fetch(st, pj >= 0 ? tile - (u64)(j - pj) : tile, w[p]);
  }
}

template <class A, int OP, int P, int SP>
UNP_DEV A lookback_finish(const u64* st, u64 tile, i64 j, int lane, u32 epoch, const waits& wt,
                          u64 (&w)[P][tile_status<A, SP>::W]) {
  typedef fold<A, OP> F;
  typedef tile_status<A, SP> S;
  const A I = F::identity();
  A excl = I;
  i64 near = j - 1 - lane;
  for (;;) {
    A v[P];
    int state[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const i64 pj = near - 64 * p;
      v[p] = I;
      state[p] = pj >= 0 ? S::decode(w[p], epoch, v[p]) : 2;
      if (pj < 0) v[p] = I;
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const i64 pj = near - 64 * p;
      if (state[p] == 0) {
        const u64 t0 = wall_clock64();
        do {
          __builtin_amdgcn_s_sleep(1);
          state[p] = S::probe(st, tile - (u64)(j - pj), epoch, v[p]);
          if (state[p] == 0 && wait_over(t0, wt)) {
            note_stall(wt);
            v[p] = I;
            state[p] = 2;
          }
        } while (state[p] == 0);
      }
      const u64 incl = __ballot(state[p] == 2);
      const int f = incl ? __builtin_ctzll(incl) : 63;
      const A c = lane <= f ? v[p] : I;
      excl = F::apply(wave_reduce<A, OP>(c), excl);
      if (incl) return excl;
    }
    near -= 64 * P;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const i64 pj = near - 64 * p;
      S::fetch(st, pj >= 0 ? tile - (u64)(j - pj) : tile, w[p]);
    }
  }
}

template <class A, int OP, int P = 1, int SP = 0>
UNP_DEV A lookback(const u64* st, u64 tile, i64 j, int lane, u32 epoch, const waits& wt) {
  u64 w[P][tile_status<A, SP>::W];
  lookback_issue<A, P, SP>(st, tile, j, lane, w);
  return lookback_finish<A, OP, P, SP>(st, tile, j, lane, epoch, wt, w);
}

// The look-back of a float fold, with an association fixed by the tiling alone.
//
// A row's tiles form groups of 64 (tile j is lane j % 64 of group j / 64).  Group k's total
// G(k) = fold(G(k-1), reduce(group k's aggregates)), with G(-1) the identity and reduce the
// wave's fixed DPP tree (wave_reduce, which is also lane 63 of wave_inclusive_scan).  The carry
// into tile j is fold(G(k-1), scan(aggregates of tiles 64k .. j-1)), scan the same tree.  No
// value depends on which block computes it or when, so the result bits are fixed for a given
// tile size, whatever the grid and the timing.
//
// G(k) is published in the status slot of the group's last tile (flag 1, over its aggregate);
// a row's first tile carries flag 1 too, where the aggregate is its own prefix.  The look-back
// probes its group's earlier tiles (window a) and the D groups before it (windows 1 .. D, all in
// one round trip).  Walking back from group k-1, it stops at the first group whose total is
// published (or past the row's first group, whose predecessor total is the identity); with every
// aggregate of the groups walked over present, it refolds their totals in order,
// G(m) = fold(G(m-1), reduce(group m)), which gives the same bits whoever computes them, and
// publishes each.  Otherwise it probes again (the lowest group without a total gets one from its
// own last tile, whose look-back waits only on lower tiles).  The last tile of a group publishes
// G(k) itself.  `agg` is this tile's aggregate.  D = 2 measured best for the f32 scan: deeper
// windows cost more probe words per look-back than the waits they save.
template <class A, int OP, int SP, int D = 2>
UNP_DEV A lookback_grouped(u64* st, u64 g, i64 j, int lane, u32 epoch, const waits& wt, A agg) {
  typedef fold<A, OP> F;
  typedef tile_status<A, SP> S;
  constexpr int W = S::W;
  const A I = F::identity();
  const i64 k = j >> 6;
  const int q = (int)(j & 63);
  const u64 row0 = g - (u64)j;  // status index of the row's first tile
  // Window a: lane l < q reads tile 64k + l; window d: lane l reads tile 64(k-d) + l.  Lanes
  // with nothing to read take the tile's own slot.
  const u64 ia = lane < q ? row0 + (u64)(64 * k + lane) : g;
  const u64 t0 = wall_clock64();
  for (;;) {
    u64 wa[W], wd[D][W];
    S::fetch(st, ia, wa);
#pragma unroll
    for (int d = 1; d <= D; ++d) S::fetch(st, k >= d ? row0 + (u64)(64 * (k - d) + lane) : g, wd[d - 1]);
    A va = I;
    const int sa = lane < q ? S::decode(wa, epoch, va) : 1;
    if (lane >= q) va = lane == 63 ? agg : I;
    // Every earlier tile of the group has published (an aggregate; flag 1 only on a row's
    // first tile, where it is the aggregate too).
    bool ok = __ballot(sa == 0) == 0;
    A vd[D];
    int depth = 0;  // groups k-1 .. k-depth+1 are folded onto the total found at k-depth
    A base = I;
    if (ok) {
#pragma unroll
      for (int d = 1; d <= D; ++d) {
        if (depth != 0) break;
        if (k < d) {
          depth = d;  // past the row's first group: G(-1) is the identity
          break;
        }
        vd[d - 1] = I;
        const int sd = S::decode(wd[d - 1], epoch, vd[d - 1]);
        if (__builtin_amdgcn_readlane(sd, 63) == 2) {
          base = readlane(vd[d - 1], 63);  // G(k-d) published
          depth = d;
        } else if (__ballot(sd == 0) != 0) {
          break;  // an aggregate of group k-d is not out yet
        }
      }
    }
    if (ok && depth != 0) {
      A gprev = base;
#pragma unroll
      for (int d = D; d >= 1; --d) {
        if (d < depth) {
          gprev = F::apply(gprev, wave_reduce<A, OP>(vd[d - 1]));
          if (lane == 0) S::publish(st, row0 + (u64)(64 * (k - d) + 63), 1, gprev, epoch);
        }
      }
      const A sc_a = wave_inclusive_scan<A, OP>(va, lane);
      const A inner = q > 0 ? readlane(sc_a, q - 1) : I;
      if (q == 63 && lane == 0) S::publish(st, g, 1, F::apply(gprev, readlane(sc_a, 63)), epoch);
      return q > 0 ? F::apply(gprev, inner) : gprev;
    }
    if (wait_over(t0, wt)) {
      if (lane == 0) note_stall(wt);
      // A group's last tile publishes a total even after giving up (the fold of what it has, with
      // no carry), so that the tiles after it stop there instead of each waiting out the bound;
      // the stall count already marks the launch's outputs invalid.
      if (q == 63) {
        const A tot = wave_reduce<A, OP>(va);
        if (lane == 0) S::publish(st, g, 1, tot, epoch);
      }
      return I;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// One wave's tile: load, tile-local scan, publish, look back, store.
// One block tile: every wave loads and scans its stripe set (WT = 64 * VEC * K positions),
// the waves' aggregates are combined in LDS, wave 0 publishes the block tile's aggregate,
// looks back and publishes its inclusive prefix, and every wave stores its prefixes.
template <class T, int OP, bool EXCL, bool REV, int VEC, int K, int WPB, int SP, bool FIXED = false>
UNP_DEV void scan_lookback(const T* __restrict__ in, T* __restrict__ out, i64 rows, i64 cols,
                           u64* __restrict__ st, u32* __restrict__ counter, u32 ticket_base,
                           u32 epoch, waits wt) {
  typedef typename acc<T, OP>::type A;
  typedef fold<A, OP> F;
  typedef tile_status<A, SP> S;
  constexpr i64 WT = (i64)64 * VEC * K;
  constexpr i64 BT = WT * WPB;
  __shared__ u32 slot[2];
  __shared__ A wagg[WPB];
  __shared__ A gbase;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const A I = F::identity();
  const T pad = (T)I;  // the identity, exactly representable at the element type
  const i64 tpr = (cols + BT - 1) / BT;
  const u64 total = (u64)rows * (u64)tpr;
  if (tid == 0)
    slot[0] = draw_ticket(counter) - ticket_base;
  __syncthreads();
  for (int r = 0;; ++r) {
    const u64 g = slot[r & 1];
    if (g >= total) break;  // uniform across the block
    u32 next = 0;
    if (tid == 0) next = draw_ticket(counter);
    const i64 row = (i64)(g / (u64)tpr);
    const i64 j = (i64)g - row * tpr;
    const i64 p0 = j * BT + (i64)wave * WT;
    const bool full = p0 + WT <= cols;
    const T* __restrict__ rin = in + row * cols;
    T* __restrict__ rout = out + row * cols;

    // Load this wave's positions, elements in scan order.
    vec<T, VEC> x[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const i64 pos = p0 + ((i64)k * 64 + lane) * VEC;
      if (full || pos + VEC <= cols) {
        if constexpr (REV) {
          const vec<T, VEC> v = ld_nt<T, VEC>(rin + (cols - VEC - pos));
#pragma unroll
          for (int e = 0; e < VEC; ++e) x[k].e[e] = v.e[VEC - 1 - e];
        } else {
          x[k] = ld_nt<T, VEC>(rin + pos);
        }
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const i64 q = pos + e;
          x[k].e[e] = q < cols ? rin[REV ? cols - 1 - q : q] : pad;
        }
      }
    }

    // Wave-local prefixes: pre[k] is the fold of this wave's elements before lane's vector k.
    A pre[K];
    A carry = I;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      A s = (A)x[k].e[0];
#pragma unroll
      for (int e = 1; e < VEC; ++e) s = F::apply(s, (A)x[k].e[e]);
      const A inc = wave_inclusive_scan<A, OP>(s, lane);
      pre[k] = F::apply(carry, wave_shr1(inc, I));
      carry = F::apply(carry, readlane(inc, 63));
    }
    if (lane == 0) wagg[wave] = carry;
    __syncthreads();

    // The fold of the earlier waves of this block tile.
    A wex = I;
    for (int w = 0; w < wave; ++w) wex = F::apply(wex, wagg[w]);
    if (wave == 0) {
      A agg = wagg[0];
#pragma unroll
      for (int w = 1; w < WPB; ++w) agg = F::apply(agg, wagg[w]);
      A gex = I;
      if (j == 0) {
        if (lane == 0) S::publish(st, g, 1, agg, epoch);
      } else {
        if (lane == 0) S::publish(st, g, 0, agg, epoch);
        if constexpr (FIXED && traits<A>::is_float) {
          gex = lookback_grouped<A, OP, SP>(st, g, j, lane, epoch, wt, agg);
        } else {
          gex = lookback<A, OP, 1, SP>(st, g, j, lane, epoch, wt);
          if (lane == 0) S::publish(st, g, 1, F::apply(gex, agg), epoch);
        }
      }
      if (lane == 0) {
        gbase = gex;
        slot[(r + 1) & 1] = next - ticket_base;
      }
    }
    __syncthreads();
    const A base = F::apply(gbase, wex);

#pragma unroll
    for (int k = 0; k < K; ++k) {
      A v = F::apply(base, pre[k]);
      vec<T, VEC> o;
      const i64 pos = p0 + ((i64)k * 64 + lane) * VEC;  // scan-order index of element 0
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        if constexpr (EXCL) {
          o.e[e] = scan_out<T, OP>(v, pos + e);
          v = F::apply(v, (A)x[k].e[e]);
        } else {
          v = F::apply(v, (A)x[k].e[e]);
          o.e[e] = scan_out<T, OP>(v, pos + e + 1);
        }
      }
      if (full || pos + VEC <= cols) {
        if constexpr (REV) {
          vec<T, VEC> v2;
#pragma unroll
          for (int e = 0; e < VEC; ++e) v2.e[e] = o.e[VEC - 1 - e];
          st_nt<T, VEC>(rout + (cols - VEC - pos), v2);
        } else {
          st_nt<T, VEC>(rout + pos, o);
        }
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const i64 q = pos + e;
          if (q < cols) rout[REV ? cols - 1 - q : q] = o.e[e];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Scans of NI inputs with a pre-map and a fused post (lift_scan_opdef with pre and post,
// kernel_lift.rs:530-602; scan_launched.rs:140-160).  At each position OPS::pre evaluates in f64
// over the position's inputs and rounds once to T, and that element is what the fold takes
// (`val = up(pre)`).  The stored prefix is rounded once to T (`red`).  With a post, OPS::post
// evaluates in f64 over `red` (r[0]) and the position's inputs (x[k]) and rounds once at the
// store.  At I32 and I64 (no post, no Mean) the pre is evaluated at T by the total integer rule
// and the fold wraps at T.  OPS::arg is the type the expressions read their inputs at.
// ---------------------------------------------------------------------------------------
template <class T, int NI, class OPS> UNP_DEV T xscan_elem(const T* const* __restrict__ in, i64 off, T (&raw)[NI]) {
  typename OPS::arg x[NI];
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    raw[k] = in[k][off];
    x[k] = (typename OPS::arg)raw[k];
  }
  return (T)OPS::pre(x);
}
template <class T, int NI, class OPS> UNP_DEV T xscan_store(T red, const T (&raw)[NI]) {
  if constexpr (OPS::has_post) {
    double x[NI], r[1] = {(double)red};
#pragma unroll
    for (int k = 0; k < NI; ++k) x[k] = (double)raw[k];
    return (T)OPS::post(r, x);
  } else {
    return red;
  }
}

// The serial lift's order (as scan_seq): one lane per column of A x S x B, bit-exact.
template <class T, int NI, int OP, class OPS, bool EXCL, bool REV>
UNP_DEV void xscan_seq(const T* const* __restrict__ in, T* __restrict__ out, i64 A, i64 S, i64 B) {
  typedef typename serial_acc<T>::type Ac;
  typedef fold<Ac, OP> F;
  const i64 cols = A * B;
  const i64 stride = (i64)gridDim.x * blockDim.x;
  for (i64 c = (i64)blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += stride) {
    const i64 a = c / B, b = c - a * B;
    const i64 base = a * S * B + b;
    Ac v = F::identity();
    for (i64 i = 0; i < S; ++i) {
      const i64 off = base + (REV ? S - 1 - i : i) * B;
      T raw[NI];
      const T e = xscan_elem<T, NI, OPS>(in, off, raw);
      if constexpr (EXCL) {
        out[off] = xscan_store<T, NI, OPS>(scan_out<T, OP>(v, i), raw);
        v = F::apply(v, (Ac)e);
      } else {
        v = F::apply(v, (Ac)e);
        out[off] = xscan_store<T, NI, OPS>(scan_out<T, OP>(v, i + 1), raw);
      }
    }
  }
}

// The device schedule (innermost axis, Sum / Max / Min, as scan_lookback with one element per
// lane per step): block tiles of WPB * 64 * K positions taken by ticket, a wave-local scan of
// the pre-mapped elements, the block's aggregate published and the row's earlier tiles folded by
// decoupled look-back, each prefix rounded once and passed through the post.  Lane l's step k
// is position k * 64 + l of its wave's stripe, so every load and store of a step is contiguous.
template <class T, int NI, int OP, class OPS, bool EXCL, bool REV, int K, int WPB, int SP, bool FIXED = false>
UNP_DEV void xscan_lookback(const T* const* __restrict__ in, T* __restrict__ out, i64 rows, i64 cols,
                            u64* __restrict__ st, u32* __restrict__ counter, u32 ticket_base, u32 epoch, waits wt) {
  typedef typename acc<T, OP>::type A;
  typedef fold<A, OP> F;
  typedef tile_status<A, SP> S;
  constexpr i64 WT = (i64)64 * K;
  constexpr i64 BT = WT * WPB;
  __shared__ u32 slot[2];
  __shared__ A wagg[WPB];
  __shared__ A gbase;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const A I = F::identity();
  const T pad = (T)I;  // the identity, exactly representable at the element type
  const i64 tpr = (cols + BT - 1) / BT;
  const u64 total = (u64)rows * (u64)tpr;
  if (tid == 0) slot[0] = draw_ticket(counter) - ticket_base;
  __syncthreads();
  for (int r = 0;; ++r) {
    const u64 g = slot[r & 1];
    if (g >= total) break;  // uniform across the block
    u32 next = 0;
    if (tid == 0) next = draw_ticket(counter);
    const i64 row = (i64)(g / (u64)tpr);
    const i64 j = (i64)g - row * tpr;
    const i64 p0 = j * BT + (i64)wave * WT;

    // This wave's elements in scan order, pre-mapped; the raw inputs kept for the post.
    T x[K];
    T raw[K][OPS::has_post ? NI : 1];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const i64 pos = p0 + (i64)k * 64 + lane;
      if (pos < cols) {
        T rk[NI];
        x[k] = xscan_elem<T, NI, OPS>(in, row * cols + (REV ? cols - 1 - pos : pos), rk);
        if constexpr (OPS::has_post) {
#pragma unroll
          for (int q = 0; q < NI; ++q) raw[k][q] = rk[q];
        }
      } else {
        x[k] = pad;
      }
    }

    // Wave-local prefixes: pre[k] is the fold of this wave's elements before lane's step k.
    A pre[K];
    A carry = I;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const A inc = wave_inclusive_scan<A, OP>((A)x[k], lane);
      pre[k] = F::apply(carry, wave_shr1(inc, I));
      carry = F::apply(carry, readlane(inc, 63));
    }
    if (lane == 0) wagg[wave] = carry;
    __syncthreads();

    A wex = I;
    for (int w = 0; w < wave; ++w) wex = F::apply(wex, wagg[w]);
    if (wave == 0) {
      A agg = wagg[0];
#pragma unroll
      for (int w = 1; w < WPB; ++w) agg = F::apply(agg, wagg[w]);
      A gex = I;
      if (j == 0) {
        if (lane == 0) S::publish(st, g, 1, agg, epoch);
      } else {
        if (lane == 0) S::publish(st, g, 0, agg, epoch);
        if constexpr (FIXED && traits<A>::is_float) {
          gex = lookback_grouped<A, OP, SP>(st, g, j, lane, epoch, wt, agg);
        } else {
          gex = lookback<A, OP, 1, SP>(st, g, j, lane, epoch, wt);
          if (lane == 0) S::publish(st, g, 1, F::apply(gex, agg), epoch);
        }
      }
      if (lane == 0) {
        gbase = gex;
        slot[(r + 1) & 1] = next - ticket_base;
      }
    }
    __syncthreads();
    const A base = F::apply(gbase, wex);

#pragma unroll
    for (int k = 0; k < K; ++k) {
      const i64 pos = p0 + (i64)k * 64 + lane;  // scan-order index
      if (pos < cols) {
        const A before = F::apply(base, pre[k]);
        const T red = EXCL ? scan_out<T, OP>(before, pos) : scan_out<T, OP>(F::apply(before, (A)x[k]), pos + 1);
        T rk[NI];
        if constexpr (OPS::has_post) {
#pragma unroll
          for (int q = 0; q < NI; ++q) rk[q] = raw[k][q];
        }
        out[row * cols + (REV ? cols - 1 - pos : pos)] = xscan_store<T, NI, OPS>(red, rk);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// LDS-staged single-pass scan with decoupled look-back, for rows whose scanned extent is a
// multiple of VEC (in / out 16-byte aligned).
//
// A block has NC consumer waves and one producer wave.  The block tile (BT = NC * 64 * VEC * K
// consecutive positions of one row) is staged in one of two LDS buffers.  Consumer wave c owns
// positions c * WT .. (WT = 64 * VEC * K); its load k of lane l is positions
// (k * 64 + l) * VEC .. + VEC, the layout one 16-byte global->LDS DMA load writes.
//
// Round r:
//   producer   draws the ticket of round r + 1, streams that tile from HBM into the other
//              buffer (DMA loads: no VGPRs hold data in flight), waits for it, folds each
//              consumer wave's share into wagg[(r + 1) & 1][c] and publishes the tile's
//              aggregate (its inclusive prefix for a row's first tile) at once;
//   consumers  scan the tile of round r out of LDS with the aggregates the producer left,
//              wave 0 looks back and publishes the inclusive prefix and hands the exclusive
//              prefix to the other waves through an LDS flag, every wave stores;
//   barrier    the only block-wide barrier: the next tile is in LDS, this one is done with.
// A tile's aggregate is out about one DMA latency after its ticket is drawn, whatever the
// consumers are doing, so a look-back seldom waits on a predecessor.  A block holds at most
// two tickets, processed in increasing order, and a tile waits only on tiles of lower ticket,
// all held by running blocks, so every wait ends.  Each block draws exactly one ticket past
// the last tile: the host advances `ticket_base` by tiles + blocks per launch.
//
// Float Sum: the producer folds a wave's share lane by lane then across the wave, the
// consumers scan it in stripe order, so the f64 carry across waves and tiles is associated
// differently from the within-stripe prefixes; every output is still one f64 fold of exactly
// its prefix, held to the declared bound.
// ---------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

// Wait until at most N vector memory operations of this wave are outstanding (gfx9
// s_waitcnt encoding: vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt left at their maximum).
template <int N> UNP_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
}
UNP_DEV void wait_vm_all() { wait_vm<0>(); }

// fn(ic<0>{}), fn(ic<1>{}), ..., fn(ic<N - 1>{}): a loop whose index is a constant expression
// in the body (for immediates such as a wait count).
template <int V> struct ic {
  static constexpr int value = V;
};
template <int N, int I = 0, class Fn> UNP_DEV void unroll_for(Fn&& fn) {
  if constexpr (I < N) {
    fn(ic<I>{});
    unroll_for<N, I + 1>(fn);
  }
}

// A block barrier that orders LDS only: no wait on outstanding global stores.  A wave with
// global->LDS DMA in flight must wait for it first (the DMA counts as LDS writes).
UNP_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <class T, int OP, bool EXCL, bool REV, int VEC, int K, int NC, int SP, bool FIXED = false>
UNP_DEV void scan_staged(const T* __restrict__ in, T* __restrict__ out, i64 rows, i64 cols,
                         u64* __restrict__ st, u32* __restrict__ counter, u32 ticket_base,
                         u32 epoch, waits wt) {
  typedef typename acc<T, OP>::type A;
  typedef fold<A, OP> F;
  typedef tile_status<A, SP> S;
  static_assert(sizeof(T) * VEC == 16, "one 16-byte DMA load per lane");
  constexpr i64 WT = (i64)64 * VEC * K;
  constexpr i64 BT = WT * NC;
  __shared__ __attribute__((aligned(16))) T buf[2][BT];
  __shared__ A wagg[2][NC];
  __shared__ u32 tk[2];
  __shared__ A gbase;
  __shared__ u32 ready;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const i64 tpr = (cols + BT - 1) / BT;
  const u64 total = (u64)rows * (u64)tpr;
  const A I = F::identity();
  const T pad = (T)I;  // the identity, exactly representable at the element type
  // The producer folds a full tile share by share as its loads land; vmcnt holds at most 63
  // outstanding loads, so the per-share waits are exact only while (NC - 1) * K stays below it.
  constexpr bool CHUNKED = (NC - 1) * K <= 63;

  if (wave == NC) {
    // ---- producer ----
    // Stage tile g into buffer b, fold each consumer wave's share and publish the aggregate.
    // A full tile (every position inside the row, uniform) takes no per-lane predicate, so
    // its DMA and LDS reads issue back to back.
    auto load = [&](const T* __restrict__ rin, i64 t0, int b, bool full) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const i64 pos = t0 + (i64)c * WT + ((i64)k * 64 + lane) * VEC;
          if (full || pos + VEC <= cols)
            __builtin_amdgcn_global_load_lds(rin + (REV ? cols - VEC - pos : pos),
                                             (lds_void*)&buf[b][c * WT + k * 64 * VEC], 16, 0, 2 /* nt */);
        }
      }
    };
    auto share = [&](i64 t0, int b, int c, bool full) {
      A s = I;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const i64 pos = t0 + (i64)c * WT + ((i64)k * 64 + lane) * VEC;
        vec<T, VEC> v = *reinterpret_cast<const vec<T, VEC>*>(&buf[b][c * WT + (k * 64 + lane) * VEC]);
        if (!full && pos + VEC > cols) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) v.e[e] = pad;
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) s = F::apply(s, (A)v.e[e]);
      }
      return s;
    };
    auto stage = [&](u64 g, int b) {
      const i64 row = (i64)(g / (u64)tpr);
      const i64 j = (i64)g - row * tpr;
      const T* __restrict__ rin = in + row * cols;
      const i64 t0 = j * BT;
      const bool full = t0 + BT <= cols;
      A agg = I;
      if (full && CHUNKED) {
        // Loads complete in issue order, so once at most (NC - 1 - c) * K of this tile's
        // NC * K loads are outstanding, wave c's share is in LDS: fold it while the rest
        // of the tile is still arriving.  The share is read with ds_read_b128 from inline
        // assembly: for an ordinary LDS read the compiler waits for every outstanding DMA load
        // of the wave first.  The LDS stores of the shares' aggregates wait for the last share.
        load(rin, t0, b, true);
        A ws[NC];
        unroll_for<NC>([&](auto cc) {
          constexpr int c = decltype(cc)::value;
          wait_vm<(NC - 1 - c) * K>();
          const u32 at = (u32)(size_t)(lds_void*)&buf[b][c * WT + lane * VEC];
          u32x4_t raw[K];
#pragma unroll
          for (int k = 0; k < K; ++k)
            asm volatile("ds_read_b128 %0, %1" : "=v"(raw[k]) : "v"(at + (u32)(k * 64 * VEC * (int)sizeof(T))) : "memory");
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          A s = I;
#pragma unroll
          for (int k = 0; k < K; ++k) {
            asm volatile("" : "+v"(raw[k]));  // no use of raw[k] moves above the wait
            const vec<T, VEC> v = __builtin_bit_cast(vec<T, VEC>, raw[k]);
#pragma unroll
            for (int e = 0; e < VEC; ++e) s = F::apply(s, (A)v.e[e]);
          }
          ws[c] = wave_reduce<A, OP>(s);
          agg = F::apply(agg, ws[c]);
        });
        if (lane == 0) {
#pragma unroll
          for (int c = 0; c < NC; ++c) wagg[b][c] = ws[c];
        }
      } else {
        if (full) load(rin, t0, b, true);
        else load(rin, t0, b, false);
        wait_vm_all();
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const A w = wave_reduce<A, OP>(full ? share(t0, b, c, true) : share(t0, b, c, false));
          if (lane == 0) wagg[b][c] = w;
          agg = F::apply(agg, w);
        }
      }
      if (lane == 0) S::publish(st, g, j == 0 ? 1 : 0, agg, epoch);
    };
    u32 t0 = 0;
    if (lane == 0) {
      t0 = draw_ticket(counter) - ticket_base;
      tk[0] = t0;
      ready = 0;
    }
    const u64 g0 = (u32)__builtin_amdgcn_readfirstlane((int)t0);
    if (g0 < total) stage(g0, 0);
    lds_barrier();  // B0
    for (int r = 0;; ++r) {
      if ((u64)tk[r & 1] >= total) break;
      u32 t = 0;
      if (lane == 0) {
        t = draw_ticket(counter) - ticket_base;
        tk[(r + 1) & 1] = t;
      }
      const u64 gn = (u32)__builtin_amdgcn_readfirstlane((int)t);
      if (gn < total) stage(gn, (r + 1) & 1);
      lds_barrier();  // B
    }
    return;
  }

  // ---- consumers ----
  lds_barrier();  // B0
  for (int r = 0;; ++r) {
    const u64 g = tk[r & 1];
    if (g >= total) break;
    const i64 row = (i64)(g / (u64)tpr);
    const i64 j = (i64)g - row * tpr;
    const i64 p0 = j * BT + (i64)wave * WT;
    const T* __restrict__ tile = &buf[r & 1][wave * WT];
    T* __restrict__ rout = out + row * cols;

    const bool full = p0 + WT <= cols;  // uniform per wave
    // With a 4-byte carry, wave 0 issues its look-back's first probes (four windows: a round of
    // tiles back) before the in-tile scan, so their round trip overlaps the scan.  An 8-byte
    // carry's probes would hold 16 more VGPRs across the scan, which then spills (measured
    // slower), so it looks back after the scan.
    // FIXED: a float fold takes lookback_grouped, whose association the tiling alone fixes.
    constexpr bool GROUPED = FIXED && traits<A>::is_float;
    constexpr int LP = sizeof(A) == 4 ? 4 : 1;
    constexpr bool EARLY = sizeof(A) == 4 && !GROUPED;
    u64 lw[LP][S::W];
    if (EARLY && wave == 0 && j > 0) lookback_issue<A, LP, SP>(st, g, j, lane, lw);
    vec<T, VEC> x[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const vec<T, VEC> v = *reinterpret_cast<const vec<T, VEC>*>(tile + (k * 64 + lane) * VEC);
      const bool in_row = full || p0 + ((i64)k * 64 + lane) * VEC + VEC <= cols;
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[k].e[e] = in_row ? v.e[REV ? VEC - 1 - e : e] : pad;
    }
    A wex = I;
    for (int w = 0; w < wave; ++w) wex = F::apply(wex, wagg[r & 1][w]);

    A pre[K];
    A carry = I;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      A s = (A)x[k].e[0];
#pragma unroll
      for (int e = 1; e < VEC; ++e) s = F::apply(s, (A)x[k].e[e]);
      const A inc = wave_inclusive_scan<A, OP>(s, lane);
      pre[k] = F::apply(carry, wave_shr1(inc, I));
      carry = F::apply(carry, readlane(inc, 63));
    }

    A gex = I;
    if (wave == 0) {
      if (j > 0) {
        // The tile's aggregate, folded as the producer folded it.
        A agg = I;
#pragma unroll
        for (int w = 0; w < NC; ++w) agg = F::apply(agg, wagg[r & 1][w]);
        if constexpr (GROUPED) {
          gex = lookback_grouped<A, OP, SP>(st, g, j, lane, epoch, wt, agg);
        } else {
          if constexpr (EARLY) gex = lookback_finish<A, OP, LP, SP>(st, g, j, lane, epoch, wt, lw);
          else gex = lookback<A, OP, 1, SP>(st, g, j, lane, epoch, wt);
          if (lane == 0) S::publish(st, g, 1, F::apply(gex, agg), epoch);
        }
      }
      if (lane == 0) {
        gbase = gex;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __hip_atomic_store(&ready, (u32)r + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    } else {
      // Wave 0's look-back is itself bounded by the wait limit: this wait allows twice that.
      if (__hip_atomic_load(&ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != (u32)r + 1) {
        const u64 t0 = wall_clock64();
        while (__hip_atomic_load(&ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != (u32)r + 1) {
          __builtin_amdgcn_s_sleep(1);
          if (wall_clock64() - t0 >= 2 * (u64)wt.ticks) {
            if (lane == 0) note_stall(wt);
            break;
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
      gex = gbase;
    }
    const A base = F::apply(gex, wex);

#pragma unroll
    for (int k = 0; k < K; ++k) {
      A v = F::apply(base, pre[k]);
      vec<T, VEC> o;
      const i64 pos = p0 + ((i64)k * 64 + lane) * VEC;  // scan-order index of element 0
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        if constexpr (EXCL) {
          o.e[e] = scan_out<T, OP>(v, pos + e);
          v = F::apply(v, (A)x[k].e[e]);
        } else {
          v = F::apply(v, (A)x[k].e[e]);
          o.e[e] = scan_out<T, OP>(v, pos + e + 1);
        }
      }
      if (full || pos + VEC <= cols) {
        if constexpr (REV) {
          vec<T, VEC> v2;
#pragma unroll
          for (int e = 0; e < VEC; ++e) v2.e[e] = o.e[VEC - 1 - e];
          st_nt<T, VEC>(rout + (cols - VEC - pos), v2);
        } else {
          st_nt<T, VEC>(rout + pos, o);
        }
      }
    }
    lds_barrier();  // B
  }
}

// ---------------------------------------------------------------------------------------
// Row gather: out[r, :] = table[clamp(ids[r]), :] with the out-of-range policy applied to
// the store (crates/unpopped/src/kernel_lift/gather.rs:184-232): Skip leaves the row,
// ZeroFill writes zero bytes, Clamp stores the clamped row.  Rows are moved as raw bytes
// in UNIT-byte pieces; one wave per output row, waves stride over rows.
//
// gfx9 counts loads and stores on one in-order counter (vmcnt), so a wait for a load also
// waits for every store issued before it.  The ids of a wave's next rows are therefore loaded
// right after this step's data loads and before its stores: the one wait per step (for the
// data) covers them, and the next step starts without a dependent round trip.  Rows of
// exactly 64 * U units move RPW at a time per wave, with no per-lane predicate.
// ---------------------------------------------------------------------------------------
template <int UNIT> struct unit_type;
template <> struct unit_type<16> { typedef u32 elem; static constexpr int n = 4; };
template <> struct unit_type<8> { typedef u32 elem; static constexpr int n = 2; };
template <> struct unit_type<4> { typedef u32 elem; static constexpr int n = 1; };
template <> struct unit_type<2> { typedef u16 elem; static constexpr int n = 1; };
template <> struct unit_type<1> { typedef u8 elem; static constexpr int n = 1; };

template <class IDX> UNP_DEV bool below_zero(IDX v) {
  if constexpr ((IDX)(-1) < (IDX)0) return v < (IDX)0;
  else return false;
}

//
// BATCH: a gather along an axis after the first (index_select, OpDef::gather with a 1-D index,
// ir.rs:3838-3876).  The output is A x NI rows of row_bytes (the axes before the gathered one, the
// gathered one, the rest as one row), the table A x src_extent rows: output row r = a * NI + i
// takes the table row a * src_extent + clamp(ids[i]).  Without BATCH, A = 1 and NI = n_rows.
template <class IDX, int POLICY, int UNIT, int THREADS, int U, int RPW, bool BATCH = false>
UNP_DEV void gather_rows(const u8* __restrict__ table, const IDX* __restrict__ ids, u8* __restrict__ out,
                         i64 n_rows, i64 row_bytes, IDX src_extent, i64 NI = 0) {
  typedef typename unit_type<UNIT>::elem E;
  constexpr int N = unit_type<UNIT>::n;
  typedef vec<E, N> V;
  constexpr int WAVES = THREADS / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const i64 units = row_bytes / UNIT;
  // The id of output row r, and the table row its clamped id `cl` names.
  auto id_at = [&](i64 r) -> IDX {
    if constexpr (BATCH) return ids[r % NI];
    else return ids[r];
  };
  auto src_row = [&](i64 r, IDX cl) -> i64 {
    if constexpr (BATCH) return (r / NI) * (i64)src_extent + (i64)cl;
    else return (i64)cl;
  };
  if (units == 64 * U) {
    // Whole rows of 64 * U units: RPW rows of a wave in flight at once (every load of the
    // RPW rows, then the next ids, then every store).  Table rows are read through the
    // caches: an id that repeats within a launch is served from L2 or the MALL.
    const i64 rstride = (i64)gridDim.x * WAVES * RPW;
    i64 r0 = ((i64)blockIdx.x * WAVES + wave) * RPW;
    IDX nxt[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) nxt[j] = r0 + j < n_rows ? id_at(r0 + j) : (IDX)0;
    for (; r0 < n_rows; r0 += rstride) {
      V v[RPW][U];
      bool take[RPW], zero[RPW];
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const IDX raw = nxt[j];
        const bool live = r0 + j < n_rows;
        const bool below = below_zero(raw);
        const bool oob = below || !(raw < src_extent);
        take[j] = live && !(oob && POLICY != OOB_CLAMP);
        zero[j] = live && oob && POLICY == OOB_ZEROFILL;
        if (take[j]) {
          const IDX cl = below ? (IDX)0 : (oob ? (IDX)(src_extent - (IDX)1) : raw);
          const E* __restrict__ src = reinterpret_cast<const E*>(table + src_row(r0 + j, cl) * row_bytes);
#pragma unroll
          for (int k = 0; k < U; ++k) v[j][k] = ld<E, N>(src + ((i64)lane + 64 * k) * N);
        }
      }
#pragma unroll
      for (int j = 0; j < RPW; ++j) nxt[j] = r0 + rstride + j < n_rows ? id_at(r0 + rstride + j) : (IDX)0;
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        E* __restrict__ dst = reinterpret_cast<E*>(out + (r0 + j) * row_bytes);
        if (take[j]) {
#pragma unroll
          for (int k = 0; k < U; ++k) st_nt<E, N>(dst + ((i64)lane + 64 * k) * N, v[j][k]);
        } else if (zero[j]) {
          V z;
          __builtin_memset(&z, 0, sizeof(V));
#pragma unroll
          for (int k = 0; k < U; ++k) st_nt<E, N>(dst + ((i64)lane + 64 * k) * N, z);
        }
      }
    }
    return;
  }
  // Any other row width: a row per wave step, U units of each lane in flight.
  const i64 rstride = (i64)gridDim.x * WAVES;
  i64 r = (i64)blockIdx.x * WAVES + wave;
  IDX next = r < n_rows ? id_at(r) : (IDX)0;
  for (; r < n_rows; r += rstride) {
    const IDX raw = next;
    const i64 rn = r + rstride;
    const bool below = below_zero(raw);
    const bool oob = below || !(raw < src_extent);
    E* __restrict__ dst = reinterpret_cast<E*>(out + r * row_bytes);
    if (oob && POLICY != OOB_CLAMP) {
      if (rn < n_rows) next = id_at(rn);
      if constexpr (POLICY == OOB_ZEROFILL) {
        V z;
        __builtin_memset(&z, 0, sizeof(V));
        for (i64 u = lane; u < units; u += 64) st_nt<E, N>(dst + u * N, z);
      }
      continue;
    }
    const IDX cl = below ? (IDX)0 : (oob ? (IDX)(src_extent - (IDX)1) : raw);
    const E* __restrict__ src = reinterpret_cast<const E*>(table + src_row(r, cl) * row_bytes);
    if (rn < n_rows) next = id_at(rn);
    for (i64 u = lane; u < units; u += 64 * U) {
      V v[U];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const i64 uu = u + 64 * k;
        if (uu < units) v[k] = ld<E, N>(src + uu * N);
      }
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const i64 uu = u + 64 * k;
        if (uu < units) st_nt<E, N>(dst + uu * N, v[k]);
      }
    }
  }
}

// A gather over storage images (the gather lift's cell, gather.rs:184-232, at every output
// coordinate): the output extents, the table's strides (its stride along the gathered axis applies
// to the clamped index), the index's strides over the output coordinates (a full-shape index, or a
// 1-D one broadcast with zero strides), the output's strides.  One lane per output element; the
// element moves as raw bits of E.
struct gather_view {
  i64 rank, axis;
  i64 ext[8], tstr[8], istr[8], ostr[8];
  i64 outs;
};

// The general gather's storage images (kernel_lift/gather.rs:35-101): the output's extents and
// strides, and every input's strides over the output coordinates (the gathered input's stride
// along `axis` applies to the clamped index); the emitted kernel evaluates the body.
struct gather_x_view {
  i64 rank, axis;
  i64 ext[8], ostr[8];
  i64 istr[8][8];
  i64 outs;
};

template <class E, class IDX, int POLICY>
UNP_DEV void gather_strided(const E* __restrict__ table, const IDX* __restrict__ ids, E* __restrict__ out,
                            const gather_view v, IDX src_extent) {
  const i64 stride = (i64)gridDim.x * blockDim.x;
  for (i64 o = (i64)blockIdx.x * blockDim.x + threadIdx.x; o < v.outs; o += stride) {
    i64 t = 0, ix = 0, oo = 0, q = o;
    for (i64 k = v.rank - 1; k >= 0; --k) {
      const i64 c = q % v.ext[k];
      q /= v.ext[k];
      if (k != v.axis) t += c * v.tstr[k];
      ix += c * v.istr[k];
      oo += c * v.ostr[k];
    }
    const IDX raw = ids[ix];
    const bool below = below_zero(raw);
    const bool oob = below || !(raw < src_extent);
    if (oob && POLICY != OOB_CLAMP) {
      if constexpr (POLICY == OOB_ZEROFILL) out[oo] = (E)0;
      continue;
    }
    const IDX cl = below ? (IDX)0 : (oob ? (IDX)(src_extent - (IDX)1) : raw);
    out[oo] = table[t + (i64)cl * v.tstr[v.axis]];
  }
}

// ---------------------------------------------------------------------------------------
// Sub-byte dequant: out[r, c] = bf16_rne((q[r, c] - z[r, c / G]) * s[r, c / G]).
// q and z are packed two 4-bit elements per byte, low nibble first (element k lives in
// byte k / 2, bits 4 * (k & 1)), flat row-major; s is f16.  The integer difference is
// exact, converting it to f32 is exact, and the product (at most 5 x 11 significant bits)
// is exact in f32, so the one rounding is the bf16 store.
// ---------------------------------------------------------------------------------------
UNP_DEV u32 bf16_rne_bits(float f) {
  const u32 b = __builtin_bit_cast(u32, f);
  if (f != f) return (b >> 16) | 0x40u;
  return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two finite f32 values to two bf16 (round to nearest even), low element first.
UNP_DEV u32 bf16x2_rne_finite(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(u32, __builtin_convertvector(v, bf16x2_t));
}

template <bool SIGNED> UNP_DEV i32 nibble_value(u32 n) {
  if constexpr (SIGNED) return (i32)(n ^ 8u) - 8;
  else return (i32)n;
}

UNP_DEV float f16_to_f32(u16 h) { return (float)__builtin_bit_cast(_Float16, h); }

// Eight consecutive elements (one dword of packed q, nibble i = element i) under one scale s
// and one zero point z, to eight bf16 (four dwords, low element first).
//   s > 0 and finite: the nibbles n are widened with v_cvt_f32_ubyte* on the bytes of
//   (q & 0x0F0F0F0F) and (q >> 4 & 0x0F0F0F0F) (an I4 nibble goes through n ^ 8, then - 8),
//   and (n - z) * s is computed as fma(n', s, -(z - off) * s): both products are exact (at most
//   5 x 11 significant bits), so the sum is the exact (n - z) * s, and it is +0 exactly when
//   the reference's (n - z) * s is (+0 times a positive s).  v_cvt_pk_bf16_f32 rounds to
//   nearest even, which is the reference's codec on finite values.
//   Otherwise (a zero, negative, infinite or NaN scale): the reference's chain literally,
//   (float)(n - z) * s, and the software codec with its NaN rule.
template <bool QS> UNP_DEV vec<u32, 4> dequant8(u32 w, float s, i32 z) {
  vec<u32, 4> o;
  if (s > 0.0f && s < __builtin_inff()) {
    const u32 flip = QS ? 0x08080808u : 0u;
    const u32 lo = (w & 0x0F0F0F0Fu) ^ flip;
    const u32 hi = ((w >> 4) & 0x0F0F0F0Fu) ^ flip;
    const float nzs = -(float)(z + (QS ? 8 : 0)) * s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = __builtin_fmaf((float)((lo >> (8 * i)) & 0xFFu), s, nzs);
      const float b = __builtin_fmaf((float)((hi >> (8 * i)) & 0xFFu), s, nzs);
      o.e[i] = bf16x2_rne_finite(a, b);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = (float)(nibble_value<QS>((w >> (8 * i)) & 15u) - z) * s;
      const float b = (float)(nibble_value<QS>((w >> (8 * i + 4)) & 15u) - z) * s;
      o.e[i] = bf16_rne_bits(a) | (bf16_rne_bits(b) << 16);
    }
  }
  return o;
}

// Fast path: cols % G == 0 and G % 8 == 0, so element e's scale and zero point are element
// e / G of their buffers (row * cols / G + col / G) and an 8-element item never straddles a
// row or a group.  A wave tile is IPL x 64 consecutive items: each q load reads 256
// contiguous bytes, each store writes 1 KiB contiguous, both streamed past the caches.
// Every load of the next tile (q, scale, zero point) is issued before this tile's stores,
// with no per-lane predicate, so the one wait per tile (the counter is in order: loads
// issued before a store do not wait for it) finds the data there.  The tail (fewer than
// IPL x 64 items) is one item per thread.
template <bool QS, bool ZS, int G, int THREADS, int IPL>
UNP_DEV void dequant4_bf16(const u8* __restrict__ q, const u16* __restrict__ sc, const u8* __restrict__ zp,
                           u16* __restrict__ out, i64 rows, i64 cols) {
  const i64 items = rows * cols / 8;
  const int lane = threadIdx.x & 63;
  constexpr int WAVES = THREADS / 64;
  const i64 nwaves = (i64)gridDim.x * WAVES;
  const u32* __restrict__ q32 = reinterpret_cast<const u32*>(q);
  constexpr i64 PER = (i64)64 * IPL;
  const i64 full = items / PER;
  u32 w[IPL];
  u16 s16[IPL];
  u8 zb[IPL];
  auto fetch = [&](i64 tile) {
    const i64 b = tile * PER + lane;
#pragma unroll
    for (int k = 0; k < IPL; ++k) w[k] = __builtin_nontemporal_load(q32 + b + 64 * k);
#pragma unroll
    for (int k = 0; k < IPL; ++k) {
      const i64 zi = ((b + 64 * k) * 8) / G;
      s16[k] = sc[zi];
      zb[k] = zp[zi >> 1];
    }
  };
  i64 t = (i64)blockIdx.x * WAVES + (threadIdx.x >> 6);
  if (t < full) fetch(t);
  for (; t < full; t += nwaves) {
    u32 cw[IPL];
    u16 cs[IPL];
    u8 cz[IPL];
#pragma unroll
    for (int k = 0; k < IPL; ++k) {
      cw[k] = w[k];
      cs[k] = s16[k];
      cz[k] = zb[k];
    }
    if (t + nwaves < full) fetch(t + nwaves);
    const i64 b = t * PER + lane;
#pragma unroll
    for (int k = 0; k < IPL; ++k) {
      const i64 it = b + 64 * k;
      const i64 zi = (it * 8) / G;
      const u32 zz = cz[k];
      const i32 z = nibble_value<ZS>((zi & 1) ? (zz >> 4) : (zz & 15u));
      st_nt<u32, 4>(reinterpret_cast<u32*>(out + it * 8), dequant8<QS>(cw[k], f16_to_f32(cs[k]), z));
    }
  }
  for (i64 it = full * PER + (i64)blockIdx.x * THREADS + threadIdx.x; it < items; it += (i64)gridDim.x * THREADS) {
    const i64 zi = (it * 8) / G;
    const u32 zz = zp[zi >> 1];
    const i32 z = nibble_value<ZS>((zi & 1) ? (zz >> 4) : (zz & 15u));
    st_nt<u32, 4>(reinterpret_cast<u32*>(out + it * 8), dequant8<QS>(q32[it], f16_to_f32(sc[zi]), z));
  }
}

// General path: any cols and G; one element per thread step, rows block-strided.
template <bool QS, bool ZS, int G, int THREADS>
UNP_DEV void dequant4_bf16_any(const u8* __restrict__ q, const u16* __restrict__ sc, const u8* __restrict__ zp,
                               u16* __restrict__ out, i64 rows, i64 cols) {
  const i64 ng = (cols + G - 1) / G;
  for (i64 r = blockIdx.x; r < rows; r += gridDim.x) {
    for (i64 c = threadIdx.x; c < cols; c += THREADS) {
      const i64 e = r * cols + c;
      const u32 qb = q[e >> 1];
      const i32 qv = nibble_value<QS>((e & 1) ? (qb >> 4) : (qb & 15u));
      const i64 zi = r * ng + c / G;
      const u32 zb = zp[zi >> 1];
      const i32 z = nibble_value<ZS>((zi & 1) ? (zb >> 4) : (zb & 15u));
      const float s = f16_to_f32(sc[zi]);
      out[e] = (u16)bf16_rne_bits((float)(qv - z) * s);
    }
  }
}

// ---------------------------------------------------------------------------------------
// The dequantizing GEMM (crates/unpopped/tests/support/dequant.rs:104-181):
//   out[r][c] = sum_k (w[r][k] - zero[r][g]) * scale[r][g] * x[k][c],  g = k / G,
// every operation an I32 that wraps, so the result is the sum in Z / 2^32.  In that ring it
// regroups exactly as
//   sum_g scale[r][g] * (P_g[r][c] - zero[r][g] * X_g[c]),
//   P_g = sum_{k in g} w[r][k] * x[k][c],   X_g[c] = sum_{k in g} x[k][c].
// With int8 activations P_g is an int8 x int8 product sum: the MFMA's.  An I32 activation is
// split into four signed byte digits: the bytes of z = (x + 0x808080) ^ 0x808080, read as int8,
// satisfy x = sum_b 2^(8 b) digit_b(z) mod 2^32 (the low three bytes are biased by 128 into
// [0, 256) and unbiased as signed bytes; the top byte's sign extension is the wrap).  Then
// P_g = sum_b 2^(8 b) P_g,b with one int8 MFMA per digit plane.
// ---------------------------------------------------------------------------------------
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// Eight packed bytes of 4-bit weights (element i in byte i / 2, low nibble first) as sixteen
// int8 in element order, sign-extended for I4.
template <bool QS> UNP_DEV i32x4 unpack16(u64 q) {
  const u32 a = (u32)q, b = (u32)(q >> 32);
  u32 lo0 = a & 0x0F0F0F0Fu, hi0 = (a >> 4) & 0x0F0F0F0Fu;
  u32 lo1 = b & 0x0F0F0F0Fu, hi1 = (b >> 4) & 0x0F0F0F0Fu;
  if constexpr (QS) {
    // n | 0xF0 where bit 3 is set: (n & 8) * 0x1E is 0xF0 and never carries out of its byte.
    lo0 |= ((lo0 & 0x08080808u) * 0x1Eu) & 0xF0F0F0F0u;
    hi0 |= ((hi0 & 0x08080808u) * 0x1Eu) & 0xF0F0F0F0u;
    lo1 |= ((lo1 & 0x08080808u) * 0x1Eu) & 0xF0F0F0F0u;
    hi1 |= ((hi1 & 0x08080808u) * 0x1Eu) & 0xF0F0F0F0u;
  }
  i32x4 r;
  r[0] = (int)__builtin_amdgcn_perm(hi0, lo0, 0x05010400u);
  r[1] = (int)__builtin_amdgcn_perm(hi0, lo0, 0x07030602u);
  r[2] = (int)__builtin_amdgcn_perm(hi1, lo1, 0x05010400u);
  r[3] = (int)__builtin_amdgcn_perm(hi1, lo1, 0x07030602u);
  return r;
}

// unpack16 without the byte interleave: lane byte p of the result holds element sigma(p) of the 16,
// sigma = 0 2 4 6, 1 3 5 7, 8 10 12 14, 9 11 13 15 (each byte's low nibbles, then its high ones).
// dqg_prep16 writes every 16-value segment of x' in the same order, so the decode kernels' dot
// products pair the same k on both sides and need no permute (1-5% faster than unpack16 there).
// The streaming kernel keeps unpack16 and dqg_prep's natural order: with unpack16n it spilled
// more and measured about 6% slower at 128 columns.
template <bool QS> UNP_DEV i32x4 unpack16n(u64 q) {
  const u32 a = (u32)q, b = (u32)(q >> 32);
  u32 lo0 = a & 0x0F0F0F0Fu, hi0 = (a >> 4) & 0x0F0F0F0Fu;
  u32 lo1 = b & 0x0F0F0F0Fu, hi1 = (b >> 4) & 0x0F0F0F0Fu;
  if constexpr (QS) {
    lo0 |= ((lo0 & 0x08080808u) * 0x1Eu) & 0xF0F0F0F0u;
    hi0 |= ((hi0 & 0x08080808u) * 0x1Eu) & 0xF0F0F0F0u;
    lo1 |= ((lo1 & 0x08080808u) * 0x1Eu) & 0xF0F0F0F0u;
    hi1 |= ((hi1 & 0x08080808u) * 0x1Eu) & 0xF0F0F0F0u;
  }
  i32x4 r;
  r[0] = (int)lo0;
  r[1] = (int)hi0;
  r[2] = (int)lo1;
  r[3] = (int)hi1;
  return r;
}

// The byte position in an x' segment of its element i: the inverse of unpack16n's sigma.
UNP_DEV constexpr int xseg_pos(int i) { return (i & 8) + ((i & 1) << 2) + ((i & 7) >> 1); }

// 4 x 4 byte transpose: byte i of out[j] is byte j of in[i].
UNP_DEV void transpose4x4(const u32 in[4], u32 out[4]) {
  const u32 t0 = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);  // in0.0 in1.0 in0.1 in1.1
  const u32 t1 = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);  // in2.0 in3.0 in2.1 in3.1
  const u32 t2 = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);  // in0.2 in1.2 in0.3 in1.3
  const u32 t3 = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);  // in2.2 in3.2 in2.3 in3.3
  out[0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
}

template <bool QS> UNP_DEV i32 nibble_at(const u8* w, i64 e) {
  const u32 b = w[e >> 1];
  return nibble_value<QS>((e & 1) ? (b >> 4) : (b & 15u));
}

// Any shape and group: one thread per output element, k in order, u32 (wrapping) arithmetic.
template <bool QS, class XT, int THREADS>
UNP_DEV void dqgemm_any(const u8* __restrict__ w, const i32* __restrict__ zero, const i32* __restrict__ scale,
                        const XT* __restrict__ x, i32* __restrict__ out, i64 R, i64 K, i64 C, i64 G) {
  const i64 ng = (K + G - 1) / G;
  for (i64 o = (i64)blockIdx.x * THREADS + threadIdx.x; o < R * C; o += (i64)gridDim.x * THREADS) {
    const i64 r = o / C, c = o - r * C;
    u32 acc = 0;
    for (i64 k = 0; k < K; ++k) {
      const i64 gi = r * ng + k / G;
      const u32 d = (u32)nibble_at<QS>(w, r * K + k) - (u32)zero[gi];
      acc += d * (u32)scale[gi] * (u32)(i32)x[k * C + c];
    }
    out[o] = (i32)acc;
  }
}

// MFMA: a block computes 64 x 64 outputs, wave (wm, wn) the 32 x 32 tile at (32 wm, 32 wn),
// with v_mfma_i32_32x32x32_i8.  XB is the activation's width in bytes (1: I8, 4: I32), G the
// group, KC the k-values staged per chunk (G % KC == 0, KC % 32 == 0).  Per chunk:
//   1. the x chunk (KC x 64 elements) is loaded coalesced, split into XB digit planes and
//      transposed 4 x 4 bytes at a time into LDS as columns (xs[plane][c][k]), so a B operand
//      is one 16-byte LDS read;
//   2. the 64 columns' digit sums (sdot4) accumulate X_g; at a group's first chunk the rows'
//      scale and zero * scale go to LDS;
//   3. each MFMA step's A operand is 8 packed bytes of the lane's row unpacked to 16 int8, its B
//      the lane's column's 16 bytes of a plane: lane group q of both holds k = 32 t + 16 q + i,
//      which the MFMA pairs byte for byte.
// At a group's end each lane rescales its 16 accumulators: total += scale * P - zero * scale * X_g.
// Needs K % G == 0, C % 4 == 0, x aligned to 4 XB bytes and w to 8 bytes.
template <bool QS, int XB, int G, int KC>
UNP_DEV void dqgemm_mfma(const u8* __restrict__ w, const i32* __restrict__ zero, const i32* __restrict__ scale,
                         const void* __restrict__ xv, i32* __restrict__ out, i64 R, i64 K, i64 C) {
  static_assert(XB == 1 || XB == 4, "I8 or I32 activations");
  static_assert(KC % 32 == 0 && G % KC == 0, "whole MFMA steps per chunk, whole chunks per group");
  constexpr int BM = 64, BN = 64, LS = KC + 16;  // LDS row stride of a column, bytes
  constexpr int NCH = G / KC;
  __shared__ __attribute__((aligned(16))) u8 xs[XB * BN * LS];
  __shared__ u32 xsum[2][BN];
  __shared__ u32 srow[2][BM], zsrow[2][BM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const i64 ntn = (C + BN - 1) / BN;
  const i64 items = ((R + BM - 1) / BM) * ntn;  // 64 x 64 tiles; blocks stride over them
  for (i64 item = blockIdx.x; item < items; item += gridDim.x) {
    // The previous item's LDS is free once every wave has passed this barrier.
    if (item != (i64)blockIdx.x) {
      __syncthreads();
    }
    const i64 tile_r = (item / ntn) * BM, tile_c = (item % ntn) * BN;
    const i64 ng = K / G;
    const int q = lane >> 5;  // lane group of the MFMA operands
    const i64 arow = tile_r + wm * 32 + (lane & 31);
    const bool arow_live = arow < R;
    const int bcol = wn * 32 + (lane & 31);  // local column of this lane's B operand
    const int cq = tid & 15, kq = tid >> 4;  // loader: columns 4 cq .. + 4, rows 4 kq + 64 p .. + 4
    const i64 c0 = tile_c + 4 * cq;
    const bool c0_live = c0 < C;
    u32 total[16];
  #pragma unroll
    for (int v = 0; v < 16; ++v) total[v] = 0;
    for (i64 g = 0; g < ng; ++g) {
      const int gb = (int)(g & 1);
      i32x16 P[XB];
  #pragma unroll
      for (int b = 0; b < XB; ++b)
  #pragma unroll
        for (int v = 0; v < 16; ++v) P[b][v] = 0;
      u32 xacc = 0;
  #pragma unroll 1
      for (int ch = 0; ch < NCH; ++ch) {
        const i64 k0 = g * G + (i64)ch * KC;
        // 1. x chunk -> digit planes, columns
  #pragma unroll
        for (int kl = 4 * kq; kl < KC; kl += 64) {
          u32 rows[XB][4];  // rows[j][i]: row i, column j (XB = 4) or the row's 4 bytes (XB = 1)
          if constexpr (XB == 1) {
            const signed char* x = static_cast<const signed char*>(xv);
  #pragma unroll
            for (int i = 0; i < 4; ++i)
              rows[0][i] = c0_live ? *reinterpret_cast<const u32*>(x + (k0 + kl + i) * C + c0) : 0u;
            u32 cols[4];
            transpose4x4(rows[0], cols);
  #pragma unroll
            for (int j = 0; j < 4; ++j) *reinterpret_cast<u32*>(xs + (4 * cq + j) * LS + kl) = cols[j];
          } else {
            const i32* x = static_cast<const i32*>(xv);
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              vec<u32, 4> r4;
              if (c0_live) r4 = *reinterpret_cast<const vec<u32, 4>*>(x + (k0 + kl + i) * C + c0);
              else r4.e[0] = r4.e[1] = r4.e[2] = r4.e[3] = 0u;
  #pragma unroll
              for (int j = 0; j < 4; ++j) rows[j][i] = (r4.e[j] + 0x00808080u) ^ 0x00808080u;
            }
  #pragma unroll
            for (int j = 0; j < 4; ++j) {
              u32 planes[4];
              transpose4x4(rows[j], planes);
  #pragma unroll
              for (int b = 0; b < 4; ++b) *reinterpret_cast<u32*>(xs + (b * BN + 4 * cq + j) * LS + kl) = planes[b];
            }
          }
        }
        // 2. the rows' scale and zero * scale (rows past R: 0), once per group
        if (ch == 0 && tid < BM) {
          const i64 r = tile_r + tid;
          const u32 sv = r < R ? (u32)scale[r * ng + g] : 0u;
          const u32 zv = r < R ? (u32)zero[r * ng + g] : 0u;
          srow[gb][tid] = sv;
          zsrow[gb][tid] = zv * sv;
        }
        __syncthreads();
        if (tid < BN) {
  #pragma unroll
          for (int b = 0; b < XB; ++b) {
            const u32* col = reinterpret_cast<const u32*>(xs + (b * BN + tid) * LS);
            int acc = 0;
  #pragma unroll 8
            for (int i = 0; i < KC / 4; ++i) acc = __builtin_amdgcn_sdot4((int)col[i], 0x01010101, acc, false);
            xacc += (u32)acc << (8 * b);
          }
          if (ch == NCH - 1) xsum[gb][tid] = xacc;
        }
        // 3. the chunk's MFMA steps
        const u8* wrow = w + (arow * K + k0) / 2;
  #pragma unroll
        for (int t = 0; t < KC / 32; ++t) {
          const u64 packed = arow_live ? *reinterpret_cast<const u64*>(wrow + (32 * t + 16 * q) / 2) : 0ull;
          const i32x4 a = unpack16<QS>(packed);
  #pragma unroll
          for (int b = 0; b < XB; ++b) {
            const i32x4 bv = *reinterpret_cast<const i32x4*>(xs + (b * BN + bcol) * LS + 32 * t + 16 * q);
            P[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bv, P[b], 0, 0, 0);
          }
        }
        __syncthreads();  // xs is free for the next chunk; xsum is written
      }
      // 4. rescale: lane's element v is row 8 (v / 4) + 4 q + v % 4 of the wave tile, column l % 32.
      // srow, zsrow and xsum alternate between two buffers by group, so the next group's writes
      // (before its first barrier) never meet this group's reads.
      const u32 xc = xsum[gb][bcol];
  #pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int lr = wm * 32 + 8 * (v >> 2) + 4 * q + (v & 3);
        u32 p = (u32)P[0][v];
  #pragma unroll
        for (int b = 1; b < XB; ++b) p += (u32)P[b][v] << (8 * b);
        total[v] += srow[gb][lr] * p - zsrow[gb][lr] * xc;
      }
    }
    const i64 c = tile_c + bcol;
    if (c < C) {
  #pragma unroll
      for (int v = 0; v < 16; ++v) {
        const i64 r = tile_r + wm * 32 + 8 * (v >> 2) + 4 * q + (v & 3);
        if (r < R) out[r * C + c] = (i32)total[v];
      }
    }
  }

}

// ---------------------------------------------------------------------------------------
// The streaming schedule for whole groups of 64-multiples (G % KC == 0, KC % 64 == 0).
//
// A pre-pass repacks x once into x' (MFMA-ready digit planes) and the group column sums:
//   x'[kc][b][kseg][c][16 bytes]: digit plane b of x[kc KC + 16 kseg + i][c], i < 16, for
//     chunk kc (KC k-values), columns c < Cp (a multiple of 64; columns past C are 0);
//   xsum[g][c] = sum_{k in g} x[k][c] (wrapping), Cp entries per group and 64 spare at the end.
// It also zeroes out when the main kernel accumulates split-K parts with atomics.
//
// The main kernel: a block owns BM = 32 WR TM rows x BN = 32 WC TN columns, TM x TN 32 x 32
// MFMA tiles per wave (a tile row's unpacked w operand serves its TN column tiles, a tile
// column's x' operand its TM row tiles), and a range
// of whole groups (split-K: parts add into out with u32 atomics, which are exact and order-free
// in Z / 2^32).  It streams the chunks of its range through NS LDS stages with global->LDS DMA:
// per chunk the w rows (each op RPO rows x SPR contiguous 16-byte segments, XOR-swizzled in
// LDS), the x' columns, the rows' scales and zero points and the group's column sums.  Each wave issues a fixed share of a stage's DMA ops; at the top of chunk i it
// waits until only its ops of the NS - 2 younger stages are outstanding, a barrier makes the
// whole stage visible and retires the stage read last, and the wave refills that stage with
// chunk i + NS - 1 (clamped to the range, so every pass issues the same ops).  No other
// vector memory operation is in flight inside the loop, so the wait counts are exact.  The
// stages are distinct __shared__ objects and the loop has no branch between a DMA and the
// reads of its stage: the compiler can then tell that a read of one stage does not depend on
// the DMA into another and inserts no wait of its own (a branch, such as waits that differ
// by wave, makes it drain every DMA once per pass of the unrolled loop).
// ---------------------------------------------------------------------------------------
template <class XT, int XB, int KC>
UNP_DEV void dqg_prep(const XT* __restrict__ x, u8* __restrict__ xp, u32* __restrict__ xsum, i64 K, i64 C,
                      i64 Cp, i64 G, i32* __restrict__ out, i64 n_out) {
  static_assert(KC % 64 == 0, "chunks of whole 16-value segments and MFMA step pairs");
  __shared__ u32 part[4][64];
  const int tid = threadIdx.x, cl = tid & 63, t4 = tid >> 6;
  const i64 slabs = Cp / 64;
  const i64 items = (K / G) * slabs;  // (group, 64-column slab); blocks stride over them
  for (i64 item = blockIdx.x; item < items; item += gridDim.x) {
    // The previous item's LDS is free once every wave has passed this barrier.
    if (item != (i64)blockIdx.x) {
      __syncthreads();
    }
    const i64 g = item / slabs, c = (item % slabs) * 64 + cl;
    const bool live = c < C;
    u32 sum = 0;
    for (i64 ks = t4; ks < G / 16; ks += 4) {
      const i64 k0 = g * G + ks * 16;
      u32 wd[XB][4];
  #pragma unroll
      for (int b = 0; b < XB; ++b)
  #pragma unroll
        for (int e = 0; e < 4; ++e) wd[b][e] = 0;
  #pragma unroll
      for (int i = 0; i < 16; ++i) {
        const u32 v = live ? (u32)(i32)x[(k0 + i) * C + c] : 0u;
        sum += v;
        const u32 z = XB == 4 ? ((v + 0x00808080u) ^ 0x00808080u) : (v & 0xFFu);
  #pragma unroll
        for (int b = 0; b < XB; ++b) wd[b][i >> 2] |= ((z >> (8 * b)) & 0xFFu) << (8 * (i & 3));
      }
      const i64 kc = k0 / KC, kseg = (k0 % KC) / 16;
  #pragma unroll
      for (int b = 0; b < XB; ++b) {
        vec<u32, 4> o;
  #pragma unroll
        for (int e = 0; e < 4; ++e) o.e[e] = wd[b][e];
        *reinterpret_cast<vec<u32, 4>*>(xp + (((kc * XB + b) * (KC / 16) + kseg) * Cp + c) * 16) = o;
      }
    }
    part[t4][cl] = sum;
    __syncthreads();
    if (t4 == 0) xsum[g * Cp + c] = part[0][cl] + part[1][cl] + part[2][cl] + part[3][cl];
  }
  for (i64 o = (i64)blockIdx.x * 256 + tid; o < n_out; o += (i64)gridDim.x * 256) out[o] = 0;
}

// A block barrier for LDS stages filled by DMA: s_barrier as a compiler memory barrier and no
// fence.  A fence would make every wave wait for all of its DMA (vmcnt(0)), including the
// stages still meant to be in flight; the caller has already waited for the stage it reads,
// and its earlier LDS reads have all returned (their values were consumed).
UNP_DEV void dma_stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int BM, int BN, int KC, int XB> struct dqg_stage {
  u8 a[BM * KC / 2];   // w: row r's 16-byte segment s at r * KC / 2 + 16 * (s ^ swz(r))
  u8 b[XB * KC * BN];  // x': plane p, segment ks, column c at ((p * KC / 16 + ks) * BN + c) * 16
  u32 s[BM];           // the rows' scales
};

template <bool QS, int XB, int G, int KC, int WR, int WC, int TM, int TN, int NS>
UNP_DEV void dqg_stream(const u8* __restrict__ w, const i32* __restrict__ zero, const i32* __restrict__ scale,
                        const u8* __restrict__ xp, const u32* __restrict__ xsum, i32* __restrict__ out, i64 R,
                        i64 K, i64 C, i64 Cp, i64 S) {
  constexpr int NW = WR * WC;
  static_assert(NW == 4 && KC % 64 == 0 && G % KC == 0 && NS >= 3 && NS <= 4, "four waves, whole chunks");
  constexpr int BM = 32 * WR * TM, BN = 32 * WC * TN;
  typedef dqg_stage<BM, BN, KC, XB> St;
  // w DMA: an op moves RPO rows x SPR contiguous 16-byte segments; the segment order inside a
  // row is XOR-swizzled by (row / FD) % SPR so that eight consecutive rows' reads of one
  // segment fall in eight distinct LDS bank groups.
  constexpr int SPR = KC / 32, RPO = 64 / SPR, FD = 16 / SPR;
  constexpr int NA = BM * KC / 2 / 1024, NB = XB * KC * BN / 1024, NSZ = BM / 64;
  static_assert(NA * 1024 == BM * KC / 2 && NB * 1024 == XB * KC * BN && NSZ * 64 == BM, "whole 64-lane ops");
  constexpr int OA = (NA + NW - 1) / NW, OB = (NB + NW - 1) / NW, OS = (NSZ + NW - 1) / NW;
  constexpr int OPW = OA + OB + OS;  // DMA ops per wave per stage
  static_assert((NS - 2) * OPW < 64, "the wait count fits vmcnt");
  __shared__ __attribute__((aligned(16))) St st0;
  __shared__ __attribute__((aligned(16))) St st1;
  __shared__ __attribute__((aligned(16))) St st2;
  __shared__ __attribute__((aligned(16))) St st3;
  St* const stages[4] = {&st0, &st1, &st2, &st3};

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave / WC, wc = wave % WC, q = lane >> 5, l32 = lane & 31;
  const i64 ng = K / G;
  const i64 tiles_r = (R + BM - 1) / BM, tiles_c = (C + BN - 1) / BN;
  const i64 units = tiles_r * S;
  // XCD-aware: consecutive blocks go to the eight XCDs in turn; the column tiles of one
  // (row tile, split) unit take consecutive slots of one XCD, so they share its L2 for w.
  const i64 xcd = (i64)blockIdx.x % 8, slot = (i64)blockIdx.x / 8;
  const i64 u = (slot / tiles_c) * 8 + xcd, ct = slot % tiles_c;
  if (u >= units) return;
  const i64 rt = u / S, split = u % S;
  const i64 tile_r = rt * BM, tile_c = ct * BN;
  const i64 g0 = ng * split / S, g1 = ng * (split + 1) / S;
  const i64 cpg = G / KC;                        // chunks per group
  const i64 c0 = g0 * cpg, n = (g1 - g0) * cpg;  // this block's chunks
  const i64 wbytes_row = K / 2;

  // A stage's DMA: every wave issues the same sequence, OA ops of w rows, OB of x' columns and
  // OS of scales (16-byte ops move 1 KiB, 4-byte ops 256 B), so every wave waits on the same
  // count with no branch.  Where a kind has fewer ops
  // than waves the extra ones repeat an op of that kind: both DMAs write the same bytes.
  auto issue_stage = [&](St* stp, i64 i) {
    const i64 chunk = c0 + (i < n ? i : n - 1);
    const i64 k0 = chunk * KC, g = k0 / G;
#pragma unroll
    for (int m = 0; m < OA; ++m) {
      const int o = (wave + NW * m) % NA;
      const int r = o * RPO + lane / SPR, seg = (lane % SPR) ^ ((r / FD) % SPR);
      const i64 row = tile_r + r < R ? tile_r + r : R - 1;
      __builtin_amdgcn_global_load_lds(w + row * wbytes_row + k0 / 2 + 16 * seg, (lds_void*)(stp->a + o * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int m = 0; m < OB; ++m) {
      const int o = (wave + NW * m) % NB, sl = o * 64 + lane, c = sl % BN, rest = sl / BN;
      const int pl = rest / (KC / 16), ks = rest % (KC / 16);
      __builtin_amdgcn_global_load_lds(xp + (((chunk * XB + pl) * (KC / 16) + ks) * Cp + tile_c + c) * 16,
                                       (lds_void*)(stp->b + o * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int m = 0; m < OS; ++m) {
      const int o = (wave + NW * m) % NSZ;
      const i64 r = tile_r + o * 64 + lane;
      const i64 row = r < R ? r : R - 1;
      __builtin_amdgcn_global_load_lds(scale + row * ng + g, (lds_void*)(stp->s + o * 64), 4, 0, 0);
    }
  };

  i32x16 P[TM][TN][XB];
  u32 total[TM][TN][16];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) total[a][t][v] = 0;
  i32x16 Z;
#pragma unroll
  for (int v = 0; v < 16; ++v) Z[v] = 0;

  auto compute = [&](const St* stp, i64 i) {
    const bool first = cpg == 1 || i % cpg == 0;  // the group's first chunk: accumulators start at 0
#pragma unroll
    for (int j = 0; j < KC / 64; ++j) {
      i32x4 a0[TM], a1[TM];
#pragma unroll
      for (int a = 0; a < TM; ++a) {
        const int r = 32 * (wr * TM + a) + l32, sg = 2 * j + q;
        const vec<u32, 4> araw =
            *reinterpret_cast<const vec<u32, 4>*>(stp->a + r * (KC / 2) + 16 * (sg ^ ((r / FD) % SPR)));
        a0[a] = unpack16<QS>((u64)araw.e[0] | ((u64)araw.e[1] << 32));
        a1[a] = unpack16<QS>((u64)araw.e[2] | ((u64)araw.e[3] << 32));
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int ks = 4 * j + 2 * q + h;
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
          for (int b = 0; b < XB; ++b) {
            const i32x4 bv =
                *reinterpret_cast<const i32x4*>(stp->b + ((b * (KC / 16) + ks) * BN + 32 * (wc * TN + t) + l32) * 16);
#pragma unroll
            for (int a = 0; a < TM; ++a)
              P[a][t][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(h ? a1[a] : a0[a], bv,
                                                                 (j == 0 && h == 0 && first) ? Z : P[a][t][b], 0, 0, 0);
          }
      }
    }
    if (cpg == 1 || (i + 1) % cpg == 0) {
      // The group ends: lane element v is row 8 (v / 4) + 4 q + v % 4 of its 32 x 32 tile.
      // The zero-point term is left to the pass after the loop.
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const int lr = 32 * (wr * TM + a) + 8 * i4 + 4 * q;
          const vec<u32, 4> s4 = *reinterpret_cast<const vec<u32, 4>*>(stp->s + lr);
#pragma unroll
          for (int t = 0; t < TN; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int v = 4 * i4 + e;
              u32 p = (u32)P[a][t][0][v];
#pragma unroll
              for (int b = 1; b < XB; ++b) p += (u32)P[a][t][b][v] << (8 * b);
              total[a][t][v] += s4.e[e] * p;
            }
        }
    }
  };

  // Prologue: chunks 0 .. NS - 2.
#pragma unroll
  for (int p = 0; p < NS - 1; ++p) issue_stage(stages[p], p);
  for (i64 i0 = 0; i0 < n; i0 += NS) {
#pragma unroll
    for (int I = 0; I < NS; ++I) {
      // Past the range the wait, the barrier and the (clamped) DMA still run, so every pass of
      // the loop issues the same memory operations and only the compute is conditional.
      const i64 i = i0 + I;
      wait_vm<(NS - 2) * OPW>();
      dma_stage_barrier();
      issue_stage(stages[(I + NS - 1) % NS], i + NS - 1);
      if (i < n) compute(stages[I], i);
    }
  }

  // The zero-point term, minus the sum over the block's groups of (scale zero)[r, g] xsum[g, c],
  // on the MFMA with 32 groups per instruction: lane (l32, q) holds groups 16 q .. 16 q + 15 of
  // its row (A) or column (B).  Both factors are split into signed byte digits: the bytes of
  // (v + 0x80808080) ^ 0x80808080 are digits d_i in [-128, 127] with sum d_i 256^i = v modulo
  // 2^32.  The digit pairs i + j = sh add into one accumulator (at most 4 x 32 products of
  // 2^14, exact), which then enters the total shifted left by 8 sh bits.
  // The loads go through buffer resources with the whole 32-bit byte offset in the range-checked
  // vector offset (the scalar offset is not range-checked, so it stays 0); the launcher checks that
  // every offset, a row tile and a 32-group step past the ends included, stays under 2^31.  Rows
  // past R and groups past ng lie past num_records and read 0.  A step's products
  // scale * zero for the block's BM rows x 32 groups are loaded coalesced (a wave instruction
  // covers two rows' 32 groups) into LDS rows of 36 words, groups past the block's last zeroed,
  // then each lane reads its row's 16 groups.  The LDS is stage memory, free once every DMA
  // has landed and every wave has left the loop.
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scale, (short)0, (int)(u32)(R * ng * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc((void*)zero, (short)0, (int)(u32)(R * ng * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc((void*)xsum, (short)0, (int)(u32)(ng * Cp * 4), 0x00020000);
  constexpr int SZW = 36, SZN = BM * 32 / (64 * NW);  // LDS row words; loads per thread per step
  // Two step buffers: the loads of the next step are issued before the current step's MFMAs.
  constexpr bool SZ_IN_STAGE = sizeof(St) >= sizeof(u32) * BM * SZW;
  __shared__ __attribute__((aligned(16))) u32 szx[SZ_IN_STAGE ? 4 : 2 * BM * SZW];
  u32* const szb0 = SZ_IN_STAGE ? reinterpret_cast<u32*>(&st0) : szx;
  u32* const szb1 = SZ_IN_STAGE ? reinterpret_cast<u32*>(&st1) : szx + BM * SZW;
  wait_vm<0>();
  __syncthreads();
  const int srow = tid / 32, sg = tid % 32;
  const int sofs = (int)(((tile_r + srow) * ng + sg) * 4);  // rows past R read 0 (past the end)
  // Column sums: lane (l32, q) of column tile t reads groups 16 q .. 16 q + 15 of its column
  // (below Cp: whole column tiles) at (16 q Cp + c) 4 + (gs + k) Cp 4.
  int cofs[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) cofs[t] = (int)((16 * q * Cp + tile_c + 32 * (wc * TN + t) + l32) * 4);
  u32 sv[SZN], zv[SZN], xv[TN][16];
  auto load_step = [&](i64 gs) {
#pragma unroll
    for (int m = 0; m < SZN; ++m) {
      const int so = (int)((gs + (i64)m * (64 * NW / 32) * ng) * 4);
      sv[m] = (u32)__builtin_amdgcn_raw_buffer_load_b32(rs, sofs + so, 0, 0);
      zv[m] = (u32)__builtin_amdgcn_raw_buffer_load_b32(rz, sofs + so, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int k = 0; k < 16; ++k) xv[t][k] = (u32)__builtin_amdgcn_raw_buffer_load_b32(rc, cofs[t] + (int)((gs + k) * Cp * 4), 0, 0);
  };
  if (g0 < g1) load_step(g0);
  int buf = 0;
#pragma unroll 1
  for (i64 gc = g0; gc < g1; gc += 32, buf ^= 1) {
    const int gl = (int)(g1 - gc < 32 ? g1 - gc : 32);  // groups of this step in range
    const u32 gmask = 0u - (u32)(sg < gl);
    u32* const szs = buf ? szb1 : szb0;
#pragma unroll
    for (int m = 0; m < SZN; ++m) szs[(m * (64 * NW / 32) + srow) * SZW + sg] = (sv[m] * zv[m]) & gmask;
    // The other buffer was last read before the previous step's barrier; this one is whole
    // after this barrier.
    __syncthreads();
    // This step's column-sum digits, before the next step's loads take over xv.
    i32x4 bd[TN][4];
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        u32 vb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          vb[e] = ((xv[t][4 * wd + e] & (0u - (u32)(16 * q + 4 * wd + e < gl))) + 0x80808080u) ^ 0x80808080u;
#pragma unroll
        for (int pl = 0; pl < 4; ++pl)
          bd[t][pl][wd] = (i32)(((vb[0] >> (8 * pl)) & 0xffu) | (((vb[1] >> (8 * pl)) & 0xffu) << 8) |
                                (((vb[2] >> (8 * pl)) & 0xffu) << 16) | ((vb[3] >> (8 * pl)) << 24));
      }
    if (gc + 32 < g1) load_step(gc + 32);
#pragma unroll
    for (int a = 0; a < TM; ++a) {
      const int lr = 32 * (wr * TM + a) + l32;
      i32x4 ad[4];
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        const vec<u32, 4> v4 = *reinterpret_cast<const vec<u32, 4>*>(szs + lr * SZW + 16 * q + 4 * wd);
        u32 vb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) vb[e] = (v4.e[e] + 0x80808080u) ^ 0x80808080u;
#pragma unroll
        for (int pl = 0; pl < 4; ++pl)
          ad[pl][wd] = (i32)(((vb[0] >> (8 * pl)) & 0xffu) | (((vb[1] >> (8 * pl)) & 0xffu) << 8) |
                             (((vb[2] >> (8 * pl)) & 0xffu) << 16) | ((vb[3] >> (8 * pl)) << 24));
      }
#pragma unroll
      for (int t = 0; t < TN; ++t) {
#pragma unroll
        for (int sh = 0; sh < 4; ++sh) {
          i32x16 acc = Z;
#pragma unroll
          for (int i = 0; i <= sh; ++i) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(ad[i], bd[t][sh - i], acc, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; ++v) total[a][t][v] -= (u32)acc[v] << (8 * sh);
        }
      }
    }
  }

#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const i64 c = tile_c + 32 * (wc * TN + t) + l32;
    if (c < C) {
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const i64 r = tile_r + 32 * (wr * TM + a) + 8 * (v >> 2) + 4 * q + (v & 3);
          if (r < R) {
            if (S == 1) out[r * C + c] = (i32)total[a][t][v];
            else __hip_atomic_fetch_add(reinterpret_cast<u32*>(out) + r * C + c, total[a][t][v], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
          }
        }
    }
  }
}

// ---------------------------------------------------------------------------------------
// The decode schedule for few columns (up to 64 for I8 activations, 128 for I32) and groups of
// whole 128-value steps: the weight stream dominates, so every wave streams its own rows of w
// straight into VGPRs, and the activations, which every wave of a block needs in full, come from LDS.
//
// dqg_prep16 repacks x once for 16-column tiles, with the layout dqg_prep writes for 64-value
// chunks but each segment in unpack16n's order: x'[kc][b][kseg][c][16 bytes], byte xseg_pos(i) =
// digit plane b of x[64 kc + 16 kseg + i][c], i < 16, for
// columns c < Cp (a multiple of 16; columns past C are 0), and xsum[g][c] = sum over group g of
// x[k][c] (wrapping).  It also zeroes out for the split-K atomics.  One block per (group, 16
// columns); thread (kseg slot, column).
//
// dqg_dec: a block of WV waves owns BM = 16 MT WV rows (MT 16-row m-tiles per wave), 16 NC columns
// (NC column tiles sharing each unpacked w operand) and a range of whole groups (a split of K, at
// most MAXG groups: the host picks S).  Per 128-deep step a lane loads 16 bytes of w for each
// m-tile (row 16 m + lane % 16, k-block lane / 16), D steps ahead, through buffer loads (a per-lane
// 32-bit offset plus a uniform step offset: no 64-bit address arithmetic in the loop), and reads
// its x' operands (16 bytes per column tile, half step and digit plane) from LDS.  The int4 pairs
// become two v_mfma_i32_16x16x64_i8 per m-tile and plane; the first MFMA of a group starts from a
// zero accumulator.  Every refill is unconditional (clamped to the last step), so each pass of
// the unrolled loop issues the same loads and the compiler's load counting stays exact across the
// back edge: a conditional refill makes it drain every load once per pass.  At a group's end
// total += scale * P - (scale * zero) * xsum, from LDS, where the block preloaded its rows'
// scales and products scale * zero and its columns' group sums.  All splits of a row tile run on
// one XCD, so their shared scale and zero-point cache lines come from that XCD's L2 once.  Splits
// add into out with u32 atomics, exact and order-free in Z / 2^32.
//
// x' in LDS (XM): 1 stages every step of the split before the main loop (one column tile of I8,
// 2 KiB a step); 2 streams it through two buffers of P steps, each pass of the main loop loading
// the next phase into VGPRs at its start and writing it to the other buffer at its end, then one
// barrier.  With x' loaded from L2 by every wave each step, as many bytes as its w at one column
// tile and two to four times as many at more columns or I32, the launches took 11-22% longer.
// ---------------------------------------------------------------------------------------
template <class XT, int XB>
UNP_DEV void dqg_prep16(const XT* __restrict__ x, u8* __restrict__ xp, u32* __restrict__ xsum, i64 K, i64 C,
                        i64 Cp, i64 G, i32* __restrict__ out, i64 n_out) {
  __shared__ u32 part[16][16];
  const int tid = threadIdx.x, cl = tid & 15, t16 = tid >> 4;
  const i64 tiles = Cp / 16;
  const i64 items = (K / G) * tiles;  // (group, 16-column tile); blocks stride over them
  for (i64 item = blockIdx.x; item < items; item += gridDim.x) {
    // The previous item's LDS is free once every wave has passed this barrier.
    if (item != (i64)blockIdx.x) {
      __syncthreads();
    }
    const i64 g = item / tiles, c = (item % tiles) * 16 + cl;
    const bool live = c < C;
    u32 sum = 0;
    for (i64 ks = t16; ks < G / 16; ks += 16) {
      const i64 k0 = g * G + ks * 16;
      u32 wd[XB][4];
  #pragma unroll
      for (int b = 0; b < XB; ++b)
  #pragma unroll
        for (int e = 0; e < 4; ++e) wd[b][e] = 0;
  #pragma unroll
      for (int i = 0; i < 16; ++i) {
        const u32 v = live ? (u32)(i32)x[(k0 + i) * C + c] : 0u;
        sum += v;
        // Signed byte digits of v (x = sum_b d_b 256^b, d_b in [-128, 127]) for I32; the byte for I8.
        const u32 z = XB == 4 ? ((v + 0x00808080u) ^ 0x00808080u) : (v & 0xFFu);
  #pragma unroll
        for (int b = 0; b < XB; ++b) wd[b][xseg_pos(i) >> 2] |= ((z >> (8 * b)) & 0xFFu) << (8 * (xseg_pos(i) & 3));
      }
      const i64 kc = k0 / 64, kseg = (k0 % 64) / 16;
  #pragma unroll
      for (int b = 0; b < XB; ++b) {
        vec<u32, 4> o;
  #pragma unroll
        for (int e = 0; e < 4; ++e) o.e[e] = wd[b][e];
        *reinterpret_cast<vec<u32, 4>*>(xp + (((kc * XB + b) * 4 + kseg) * Cp + c) * 16) = o;
      }
    }
    part[t16][cl] = sum;
    __syncthreads();
    if (t16 == 0) {
      u32 t = 0;
  #pragma unroll
      for (int j = 0; j < 16; ++j) t += part[j][cl];
      xsum[g * Cp + c] = t;
    }
  }
  for (i64 o = (i64)blockIdx.x * 256 + tid; o < n_out; o += (i64)gridDim.x * 256) out[o] = 0;
}

typedef unsigned int u32x4b __attribute__((ext_vector_type(4)));

template <bool QS, int XB, int G, int MT, int NC, int D, int MAXG, int WV, int XM, int P>
UNP_DEV void dqg_dec(const u8* __restrict__ w, const i32* __restrict__ zero, const i32* __restrict__ scale,
                     const u8* __restrict__ xp, const u32* __restrict__ xsum, i32* __restrict__ out, i64 R, i64 K,
                     i64 C, i64 Cp, i64 S) {
  constexpr int THREADS = 64 * WV, BM = 16 * MT * WV, BN = 16 * NC, SPG = G / 128;
  static_assert(G % 128 == 0 && D % SPG == 0, "whole steps per group, whole groups per unrolled pass");
  static_assert(XM == 1 || (XM == 2 && P % D == 0), "x' staged whole, or in phases of whole unrolled passes");
  __shared__ __attribute__((aligned(16))) u32 ss[MAXG][BM + 4];
  __shared__ __attribute__((aligned(16))) u32 zs[MAXG][BM + 4];
  __shared__ u32 xs[MAXG][BN];
  // x' in LDS as 16-byte units (step, column tile t, plane b, half-step segment e (0..7), column),
  // the column fastest: XM 1 holds every step of the block's groups; XM 2 two buffers of P steps,
  // phase f (steps f P .. f P + P - 1) in buffer f & 1.
  constexpr int XSEG = NC * XB * 8;                        // 256-byte slabs per step
  constexpr int XSTEPS = XM == 1 ? MAXG * SPG : 2 * P;     // steps the LDS holds
  __shared__ __attribute__((aligned(16))) u8 xl[XSTEPS * XSEG * 256];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = lane >> 4, r16 = lane & 15;
  const i64 ng = K / G;
  const i64 tiles_r = (R + BM - 1) / BM, tiles_c = (C + BN - 1) / BN;
  // Block b: XCD b % 8; its slot b / 8 names (row tile of that XCD, split, column tile).
  const i64 items = (tiles_r + 7) / 8 * 8 * S * tiles_c;  // XCD-interleaved (row tile, split, column tile)
  for (i64 item = blockIdx.x; item < items; item += gridDim.x) {
    // The previous item's LDS is free once every wave has passed this barrier.
    if (item != (i64)blockIdx.x) {
      __syncthreads();
    }
    const i64 xcd = item % 8, slot = item / 8, per = S * tiles_c;
    const i64 rt = (slot / per) * 8 + xcd, split = (slot % per) / tiles_c, ct = slot % tiles_c;
    if (rt >= tiles_r) continue;
    const i64 tile_r = rt * BM, tile_c = ct * BN;
    const i64 g0 = ng * split / S, g1 = ng * (split + 1) / S;
    const int ngr = (int)(g1 - g0);  // at most MAXG: the host picks S
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, (int)(u32)(R * (K / 2)), 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)xp, (short)0, (int)(u32)(K * Cp * XB), 0x00020000);
    const i64 kb = g0 * G, nsteps = (i64)ngr * SPG;
    u32 wofs[MT];
  #pragma unroll
    for (int m = 0; m < MT; ++m) {
      const i64 row = tile_r + wave * 16 * MT + 16 * m + r16;
      wofs[m] = (u32)((row < R ? row : R - 1) * (K / 2) + kb / 2 + 16 * kq);
    }
    u32x4b wv[D][MT];
    auto load = [&](int sl, i64 i) {
      const int sw = (int)(64 * i);
  #pragma unroll
      for (int m = 0; m < MT; ++m) wv[sl][m] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)wofs[m], sw, 0);
    };
    // The 16-byte x' units of `steps` steps from step s0 on (unit u: column u % 16, segment
    // (u / 16) % 8, plane, column tile, then step), steps past the block's last clamped to it.
    constexpr int UPS = XSEG * 16;  // units per step
    auto xunit = [&](i64 s0, int u) -> u32x4b {
      const int c = u % 16, e = (u / 16) % 8, b = (u / 128) % XB, t = (u / (128 * XB)) % NC;
      const i64 s = s0 + u / UPS, i = s < nsteps ? s : nsteps - 1;
      const int off = (int)((((kb / 64 + 2 * i + e / 4) * XB + b) * 4 + e % 4) * Cp + tile_c + 16 * t + c) * 16;
      return __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
    };
    // Step i's x' operand of column tile t, plane b, half step h (half step h of lane (kq, c) covers
    // k = 32 kq + 16 h + [0, 16) of the step: segment 2 kq + h).
    auto xop = [&](i64 i, int t, int b, int h) -> i32x4 {
      const i64 st = XM == 1 ? i : (i / P & 1) * P + i % P;
      return *reinterpret_cast<const i32x4*>(xl + ((((st * NC + t) * XB + b) * 8 + 2 * kq + h) * 16 + r16) * 16);
    };
  #pragma unroll
    for (int p = 0; p < D; ++p) load(p, p < nsteps ? p : nsteps - 1);
    // XM 1: every step's x' now.  XM 2: phase 0 now, each later phase while the one before runs.
    constexpr int PU = ((XM == 1 ? MAXG * SPG : P) * UPS + THREADS - 1) / THREADS;
    u32x4b tmp[PU];
    auto xfetch = [&](i64 s0, int nu) {
  #pragma unroll
      for (int j = 0; j < PU; ++j) {
        const int u = tid + THREADS * j;
        if (XM == 2 || u < nu) tmp[j] = xunit(s0, u < nu ? u : 0);
      }
    };
    auto xstore = [&](int buf, int nu) {
  #pragma unroll
      for (int j = 0; j < PU; ++j) {
        const int u = tid + THREADS * j;
        if (u < nu) *reinterpret_cast<u32x4b*>(xl + 16 * (buf * P * UPS + u)) = tmp[j];
      }
    };
    if constexpr (XM == 1) {
      xfetch(0, (int)nsteps * UPS);
      xstore(0, (int)nsteps * UPS);
    } else {
      xfetch(0, P * UPS);
      xstore(0, P * UPS);
    }
    // The preload: every load issued at once, while the first steps are in flight.
    constexpr int PL = (BM * MAXG + THREADS - 1) / THREADS, PX = (BN * MAXG + THREADS - 1) / THREADS;
    u32 sv[PL], zv[PL], cv[PX];
  #pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int idx = tid + THREADS * j, r = idx / MAXG, gg = idx % MAXG;
      const i64 row = tile_r + r < R ? tile_r + r : R - 1;
      const bool ok = r < BM && gg < ngr;
      sv[j] = ok ? (u32)scale[row * ng + g0 + gg] : 0u;
      zv[j] = ok ? (u32)zero[row * ng + g0 + gg] : 0u;
    }
  #pragma unroll
    for (int j = 0; j < PX; ++j) {
      const int idx = tid + THREADS * j, gg = idx / BN, c = idx % BN;
      cv[j] = gg < ngr ? xsum[(g0 + gg) * Cp + tile_c + c] : 0u;
    }
  #pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int idx = tid + THREADS * j, r = idx / MAXG, gg = idx % MAXG;
      if (r < BM) {
        ss[gg][r] = sv[j];
        zs[gg][r] = sv[j] * zv[j];
      }
    }
  #pragma unroll
    for (int j = 0; j < PX; ++j) {
      const int idx = tid + THREADS * j, gg = idx / BN, c = idx % BN;
      if (gg < MAXG) xs[gg][c] = cv[j];
    }
    __syncthreads();
    i32x4 Pa[MT][NC][XB];
    u32 total[MT][NC][4];
  #pragma unroll
    for (int m = 0; m < MT; ++m)
  #pragma unroll
      for (int t = 0; t < NC; ++t)
  #pragma unroll
        for (int v = 0; v < 4; ++v) total[m][t][v] = 0;
    const i32x4 Z = {0, 0, 0, 0};
    // Step i (I its place in the unrolled pass, whose start is a whole number of groups): the MFMAs
    // of w slot I % D, and at a group's end total += scale * P - (scale * zero) * xsum.
    auto step = [&](int I, i64 i) {
      const int sl = I % D;
  #pragma unroll
      for (int m = 0; m < MT; ++m) {
        const i32x4 a0 = unpack16n<QS>((u64)wv[sl][m][0] | ((u64)wv[sl][m][1] << 32));
        const i32x4 a1 = unpack16n<QS>((u64)wv[sl][m][2] | ((u64)wv[sl][m][3] << 32));
  #pragma unroll
        for (int t = 0; t < NC; ++t)
  #pragma unroll
          for (int b = 0; b < XB; ++b) {
            Pa[m][t][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, xop(i, t, b, 0), I % SPG == 0 ? Z : Pa[m][t][b], 0, 0, 0);
            Pa[m][t][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, xop(i, t, b, 1), Pa[m][t][b], 0, 0, 0);
          }
      }
      if ((I + 1) % SPG == 0) {
        // Lane (kq, c) holds rows 4 kq + v of each m-tile, column c.
        const int gg = (int)(i / SPG);
  #pragma unroll
        for (int m = 0; m < MT; ++m) {
          const int lr = wave * 16 * MT + 16 * m + 4 * kq;
          const vec<u32, 4> s4 = *reinterpret_cast<const vec<u32, 4>*>(&ss[gg][lr]);
          const vec<u32, 4> z4 = *reinterpret_cast<const vec<u32, 4>*>(&zs[gg][lr]);
  #pragma unroll
          for (int t = 0; t < NC; ++t) {
            const u32 xc = xs[gg][16 * t + r16];
  #pragma unroll
            for (int v = 0; v < 4; ++v) {
              u32 p = (u32)Pa[m][t][0][v];
  #pragma unroll
              for (int b = 1; b < XB; ++b) p += (u32)Pa[m][t][b][v] << (8 * b);
              total[m][t][v] += s4.e[v] * p - z4.e[v] * xc;
            }
          }
        }
      }
    };
    if constexpr (XM == 1) {
      for (i64 i0 = 0; i0 < nsteps; i0 += D) {
  #pragma unroll
        for (int I = 0; I < D; ++I) {
          const i64 i = i0 + I;
          if (i < nsteps) step(I, i);
          load(I, i + D < nsteps ? i + D : nsteps - 1);
        }
      }
    } else {
      // One phase per pass: the next phase's x' is loaded at the pass's start and written to the
      // other buffer at its end (whose last readers passed the previous pass's barrier), then one
      // barrier.  Every load is unconditional (clamped), so each pass issues the same loads.
      for (i64 i0 = 0; i0 < nsteps; i0 += P) {
        xfetch(i0 + P, P * UPS);
  #pragma unroll
        for (int I = 0; I < P; ++I) {
          const i64 i = i0 + I;
          if (i < nsteps) step(I, i);
          load(I % D, i + D < nsteps ? i + D : nsteps - 1);
        }
        xstore((int)((i0 / P + 1) & 1), P * UPS);
        __syncthreads();
      }
    }
  #pragma unroll
    for (int t = 0; t < NC; ++t) {
      const i64 c = tile_c + 16 * t + r16;
      if (c < C) {
  #pragma unroll
        for (int m = 0; m < MT; ++m)
  #pragma unroll
          for (int v = 0; v < 4; ++v) {
            const i64 r = tile_r + wave * 16 * MT + 16 * m + 4 * kq + v;
            if (r < R) {
              if (S == 1) out[r * C + c] = (i32)total[m][t][v];
              else __hip_atomic_fetch_add(reinterpret_cast<u32*>(out) + r * C + c, total[m][t][v], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
            }
          }
      }
    }
  }

}

// ---------------------------------------------------------------------------------------
// Access::RowReduce (crates/unpopped/src/ir.rs:2114-2125): per row, NS staged folds, each over
// a pre expression that may read the inputs and the earlier stages, then a full-width epilogue
// (softmax, RMSNorm, a centred quotient ...).
//
// Numerics follow the lifted kernel as the reference's kernel evaluator runs it
// (crates/unpopped/src/oracle/kernel_eval.rs:765-770, 924-955): a float expression is evaluated
// in f64 from its operands and rounded once per statement.  So a stage folds
// (f64)(T)pre(x, red) into an f64 accumulator (Max/Min with the NaN rule), finalises (Mean
// divides by the row length; an empty row leaves the accumulator's starting 0), and rounds
// once to T; the epilogue is evaluated in f64 over the inputs and the rounded stage values and
// rounded once at the store.  The emitted source supplies OPS: `op[S]`, `pre<S>(x, r)` and
// `epi(x, r)` over doubles, with the scalar functions below.
//
// One block per row (rows block-strided).  R > 0: the row is read once into registers
// (R vectors of VEC per thread and input, cols <= THREADS * VEC * R), and the block's next row
// is loaded into a second register set while this one runs; R == 0: each pass reads the row
// again (the later passes hit in L2).  OPS::cached names a stage whose pre value
// recurs in the epilogue (softmax's exp(x - max)): with the row in registers its f64 value per
// element is kept from the stage and OPS::epi_c reads it back in place of a second
// evaluation, which is the same f64 expression of the same operands.  Inside a pass thread t folds its positions in
// ascending order; waves combine by DPP, then in wave order, so the order is fixed by the
// geometry.
// ---------------------------------------------------------------------------------------
namespace xf {
// UnaryOp / BinaryOp in f64, as crates/unpopped/src/oracle/scalar_ops.rs:14-80, 90-150 define
// them.  Sign and Step decide on the argument rounded to the compute dtype T first
// (expr_eval.rs:130-137).
UNP_DEV double sqr(double x) { return x * x; }
UNP_DEV double rsqrt(double x) { return 1.0 / sqrt(x); }
UNP_DEV double recip(double x) { return 1.0 / x; }
UNP_DEV double sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }
UNP_DEV double relu(double x) { return x < 0.0 ? 0.0 : x; }
UNP_DEV double silu(double x) { return x * (1.0 / (1.0 + exp(-x))); }
UNP_DEV double gelu(double x) { return 0.5 * x * (1.0 + erf(x * 0.70710678118654752440)); }
UNP_DEV double atanh_odd(double x) { return copysign(atanh(fabs(x)), x); }
template <class T> UNP_DEV double sign(double x) {
  const double c = (double)(T)x;
  return c > 0.0 ? 1.0 : (c < 0.0 ? -1.0 : 0.0);
}
template <class T> UNP_DEV double step(double x) { return (double)(T)x > 0.0 ? 1.0 : 0.0; }
// NaN-propagating, and `a` on ties.
UNP_DEV double max_prop(double a, double b) { return a != a ? a : (b != b ? b : (a >= b ? a : b)); }
UNP_DEV double min_prop(double a, double b) { return a != a ? a : (b != b ? b : (a <= b ? a : b)); }
// Floored remainder (sign of the divisor).
UNP_DEV double rem_floor(double a, double b) { return a - floor(a / b) * b; }
UNP_DEV double select(double c, double a, double b) { return c != 0.0 ? a : b; }
}  // namespace xf

namespace xi {
// Integer arithmetic at I32, I64, U32 and U64 by the total rule of the reference's kernel
// evaluator (oracle/kernel_eval.rs:1114-1175, docs/int-div-shift-semantics.md rules 1-3).  Add,
// Sub and Mul wrap: they run on the unsigned type of the width and convert back.  A zero divisor
// gives the dividend; so does signed MIN / -1 (a signed divisor of -1 is the wrapping negation,
// which is the quotient for every other dividend).  A shift count's bits are read as unsigned and
// taken modulo the width (32, or 64 for a 64-bit type); Shl shifts the unsigned bits (no overflow
// for a negative or large value), Shr is arithmetic on a signed type and logical on an unsigned
// one.  Min, Max and the bitwise ops act on the type's values.
template <class T> struct ibits;
template <> struct ibits<int> { using U = unsigned int; static constexpr bool sgn = true; static constexpr unsigned w = 32; };
template <> struct ibits<unsigned int> { using U = unsigned int; static constexpr bool sgn = false; static constexpr unsigned w = 32; };
template <> struct ibits<long long> { using U = unsigned long long; static constexpr bool sgn = true; static constexpr unsigned w = 64; };
template <> struct ibits<unsigned long long> {
  using U = unsigned long long;
  static constexpr bool sgn = false;
  static constexpr unsigned w = 64;
};
template <class T> UNP_DEV T add(T a, T b) { using U = typename ibits<T>::U; return (T)((U)a + (U)b); }
template <class T> UNP_DEV T sub(T a, T b) { using U = typename ibits<T>::U; return (T)((U)a - (U)b); }
template <class T> UNP_DEV T mul(T a, T b) { using U = typename ibits<T>::U; return (T)((U)a * (U)b); }
template <class T> UNP_DEV T div(T a, T b) {
  using U = typename ibits<T>::U;
  if (b == (T)0) return a;
  if constexpr (ibits<T>::sgn) {
    if (b == (T)-1) return (T)((U)0 - (U)a);
  }
  return (T)(a / b);
}
template <class T> UNP_DEV unsigned count(T c) { return (unsigned)((typename ibits<T>::U)c & (ibits<T>::w - 1u)); }
template <class T> UNP_DEV T shl(T a, T c) { using U = typename ibits<T>::U; return (T)((U)a << count(c)); }
template <class T> UNP_DEV T shr(T a, T c) { return (T)(a >> count(c)); }
template <class T> UNP_DEV T min(T a, T b) { return a < b ? a : b; }
template <class T> UNP_DEV T max(T a, T b) { return a > b ? a : b; }
template <class T> UNP_DEV T bit_and(T a, T b) { return (T)(a & b); }
template <class T> UNP_DEV T bit_or(T a, T b) { return (T)(a | b); }
template <class T> UNP_DEV T bit_xor(T a, T b) { return (T)(a ^ b); }
}  // namespace xi

template <class T, int NI, int NS, class OPS, int THREADS, int VEC, int R, int S>
UNP_DEV void rr_stage(const T* const* rin, const vec<T, VEC> (&xr)[NI][R > 0 ? R : 1], i64 cols, double (&red)[NS],
                      double* part, double* redsh, double (&cv)[R > 0 ? R : 1][VEC]) {
  if constexpr (S < NS) {
    constexpr int OP = OPS::op[S];
    typedef fold<double, OP> F;
    constexpr int WAVES = THREADS / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const i64 nvec = cols / VEC;
    double acc = F::identity();
    auto fold_vec = [&](const vec<T, VEC> (&v)[NI]) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        double x[NI];
#pragma unroll
        for (int k = 0; k < NI; ++k) x[k] = (double)v[k].e[e];
        acc = F::apply(acc, (double)(T)OPS::template pre<S>(x, red));
      }
    };
    if constexpr (R > 0 && S == OPS::cached) {
      // This stage's per-element value recurs in the epilogue: keep it (in f64, before the
      // stage's rounding to T) for the epilogue to read back.
#pragma unroll
      for (int q = 0; q < R; ++q)
        if ((i64)q * THREADS + tid < nvec) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            double x[NI];
#pragma unroll
            for (int k = 0; k < NI; ++k) x[k] = (double)xr[k][q].e[e];
            const double p = OPS::template pre<S>(x, red);
            cv[q][e] = p;
            acc = F::apply(acc, (double)(T)p);
          }
        }
    } else if constexpr (R > 0) {
#pragma unroll
      for (int q = 0; q < R; ++q)
        if ((i64)q * THREADS + tid < nvec) {
          vec<T, VEC> xv[NI];
#pragma unroll
          for (int k = 0; k < NI; ++k) xv[k] = xr[k][q];
          fold_vec(xv);
        }
    } else {
      for (i64 v = tid; v < nvec; v += THREADS) {
        vec<T, VEC> xv[NI];
#pragma unroll
        for (int k = 0; k < NI; ++k) xv[k] = ld<T, VEC>(rin[k] + v * VEC);
        fold_vec(xv);
      }
    }
    acc = wave_reduce<double, OP>(acc);
    if (lane == 0) part[wave] = acc;
    __syncthreads();
    if (tid == 0) {
      double a = part[0];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) a = F::apply(a, part[w]);
      double fin = a;
      if constexpr (OP == OP_MEAN) fin = a / (double)cols;
      if constexpr (OP == OP_MAX || OP == OP_MIN) fin = cols == 0 ? 0.0 : a;
      redsh[S] = (double)(T)fin;
    }
    __syncthreads();
    red[S] = redsh[S];
    rr_stage<T, NI, NS, OPS, THREADS, VEC, R, S + 1>(rin, xr, cols, red, part, redsh, cv);
  }
}

template <class T, int NI, int NS, class OPS, int THREADS, int VEC, int R>
UNP_DEV void row_reduce_staged(const T* const* in, T* __restrict__ out, i64 rows, i64 cols) {
  __shared__ double part[THREADS / 64];
  __shared__ double redsh[NS];
  const int tid = threadIdx.x;
  const i64 nvec = cols / VEC;
  typedef vec<T, VEC> RowRegs[NI][R > 0 ? R : 1];
  // With the row in registers (R > 0: 16-byte vectors, cols a multiple of VEC) every load and
  // store of a row is a buffer access whose range is the row: a lane past the row's end reads 0
  // and its store is dropped, and a row past the last has an empty range.  So each row issues
  // the same R loads per input and R stores whatever its length, the compiler can count them, and
  // a wait for this row's vectors leaves the next row's loads in flight.
  auto row_rsrc = [&](const T* base, i64 row) {
    const bool live = row < rows;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (live ? row : 0) * cols), (short)0,
                                             (int)(u32)(live ? cols * (i64)sizeof(T) : 0), 0x00020000);
  };
  auto load_row = [&](i64 row, RowRegs& xr) {
    if constexpr (R > 0) {
      static_assert(sizeof(T) * VEC == 16, "the in-register rows move 16-byte vectors");
#pragma unroll
      for (int k = 0; k < NI; ++k) {
        const __amdgpu_buffer_rsrc_t rk = row_rsrc(in[k], row);
#pragma unroll
        for (int q = 0; q < R; ++q)
          xr[k][q] = __builtin_bit_cast(vec<T, VEC>, __builtin_amdgcn_raw_buffer_load_b128(rk, (q * THREADS + tid) * 16, 0, 2));
      }
    }
  };
  auto one_row = [&](i64 row, const RowRegs& xr) {
    const T* rin[NI];
#pragma unroll
    for (int k = 0; k < NI; ++k) rin[k] = in[k] + row * cols;
    T* __restrict__ rout = out + row * cols;
    double red[NS];
    double cv[R > 0 ? R : 1][VEC];
    rr_stage<T, NI, NS, OPS, THREADS, VEC, R, 0>(rin, xr, cols, red, part, redsh, cv);
    auto emit = [&](const vec<T, VEC> (&v)[NI], i64 at) {
      vec<T, VEC> o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        double x[NI];
#pragma unroll
        for (int k = 0; k < NI; ++k) x[k] = (double)v[k].e[e];
        o.e[e] = (T)OPS::epi(x, red);
      }
      st_nt<T, VEC>(rout + at * VEC, o);
    };
    if constexpr (R > 0) {
      // Lanes past the row's end compute on what they hold and their stores are dropped.
      const __amdgpu_buffer_rsrc_t ro = row_rsrc(out, row);
#pragma unroll
      for (int q = 0; q < R; ++q) {
        vec<T, VEC> o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          double x[NI];
#pragma unroll
          for (int k = 0; k < NI; ++k) x[k] = (double)xr[k][q].e[e];
          if constexpr (OPS::cached >= 0) o.e[e] = (T)OPS::epi_c(x, red, cv[q][e]);
          else o.e[e] = (T)OPS::epi(x, red);
        }
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4b, o), ro, (q * THREADS + tid) * 16, 0, 2);
      }
    } else {
      for (i64 v = tid; v < nvec; v += THREADS) {
        vec<T, VEC> xv[NI];
#pragma unroll
        for (int k = 0; k < NI; ++k) xv[k] = ld<T, VEC>(rin[k] + v * VEC);
        emit(xv, v);
      }
    }
  };
  const i64 G = gridDim.x;
  if constexpr (R > 0) {
    // Two register sets, the loop unrolled by two: the block's next row is loaded into the other
    // set before this row's stages run, so its loads are in flight under this row's arithmetic and
    // no copy between the sets waits on them.
    RowRegs xa, xb;
    load_row(blockIdx.x, xa);
    for (i64 row = blockIdx.x; row < rows; row += 2 * G) {
      load_row(row + G, xb);
      one_row(row, xa);
      if (row + G >= rows) break;
      load_row(row + 2 * G, xa);
      one_row(row + G, xb);
    }
  } else {
    RowRegs none;
    for (i64 row = blockIdx.x; row < rows; row += G) one_row(row, none);
  }
}

}  // namespace unp
