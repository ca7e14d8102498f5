// common.hpp — shared definitions of the MI355X token-loop library (libmitok).
//
// Complex<f64> is stored as HIP double2 {x = re, y = im}: the same 16-byte
// #[repr(C)] {re, im} layout as num-complex 0.4.6, so host buffers from the
// reference cross the C ABI without conversion.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mitok {

// ---- launch timing ----
// When a timing scope is armed (mitok_timing_enable), the next product or
// attention launch stamps these events at its own start and end through the
// dispatch (hipExtLaunchKernelGGL): the kernel's execution time, as a profiler
// reports it, without the cost of separate event records.  Other launches are
// plain.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
};
inline LaunchTiming& launch_timing() {
  static thread_local LaunchTiming t;
  return t;
}
#define MITOK_LAUNCH(kern, grid, block, shm, st, ...)                                         \
  do {                                                                                       \
    ::mitok::LaunchTiming& lt_ = ::mitok::launch_timing();                                    \
    if (lt_.start) {                                                                         \
      hipExtLaunchKernelGGL(kern, grid, block, shm, st, lt_.start, lt_.stop, 0, __VA_ARGS__); \
      lt_.start = lt_.stop = nullptr;                                                        \
    } else {                                                                                 \
      hipLaunchKernelGGL(kern, grid, block, shm, st, __VA_ARGS__);                           \
    }                                                                                        \
  } while (0)

// accumulator of v_mfma_f64_16x16x4f64 (4 doubles per lane)
typedef double v4d __attribute__((ext_vector_type(4)));
typedef double v2d __attribute__((ext_vector_type(2)));



// ---- status codes (include/mitok.h) ----
enum Status : int {
  OK = 0,
  ERR_ARG = 1,
  ERR_HIP = 2,
  ERR_STATE = 3,
  ERR_NAN = 4,
  ERR_NOMEM = 5,
};

// ---- device error word bits, set by kernels, read by the host after a step ----
enum ErrBits : uint32_t {
  EB_GELU_NAN = 1u,      // gelu_complex panics on NaN (utils/activation.rs:207-209)
  EB_FFN_NONFINITE = 2u, // check_nan_or_inf_3d after the FFN (transformer_network.rs:408)
  EB_BAD_TOKEN = 4u,     // id >= vocab: no embedding (embedding_layer.rs:305)
  EB_ARGMAX_NAN = 8u,    // greedy_decoding partial_cmp().unwrap() (sampling_methods.rs:12)
  EB_CTX_OVERFLOW = 16u, // a cached sequence outgrew max_ctx
  EB_BARRIER = 32u,      // a grid barrier of the resident decode loop timed out
  EB_TRAIN_NONFINITE = 64u, // a non-finite embedding gradient or row (embedding_layer.rs:242-250)
};

// ---- counter generator (identical to oracle.c / seeded.py) ----
__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t stream_key(uint64_t seed, uint64_t stream) { return mix64(mix64(seed) ^ stream); }
// uniform on [-lim, lim): (2u - 1) is exact, the product is the only rounding
__host__ __device__ inline double uniform_from_key(uint64_t key, uint64_t index, double lim) {
  double u = (double)(mix64(key ^ index) >> 11) * 0x1.0p-53;
  return (2.0 * u - 1.0) * lim;
}
inline uint64_t stream_id(uint32_t layer, uint32_t slot) { return ((uint64_t)layer << 12) | slot; }

// ---- num-complex 0.4.6 arithmetic on double2 ----
__device__ __forceinline__ double2 cadd(double2 a, double2 b) { return make_double2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ double2 csub(double2 a, double2 b) { return make_double2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ double2 cmul(double2 a, double2 b) {
  return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ double2 cscale(double2 a, double t) { return make_double2(a.x * t, a.y * t); }
__device__ __forceinline__ double2 cunscale(double2 a, double t) { return make_double2(a.x / t, a.y / t); }
// impl Div for Complex: (a * conj(b)) / norm_sqr(b)
__device__ __forceinline__ double2 cdiv(double2 a, double2 b) {
  double n = b.x * b.x + b.y * b.y;
  return make_double2((a.x * b.x + a.y * b.y) / n, (a.y * b.x - a.x * b.y) / n);
}
// Complex::sqrt: positive-real / imaginary-axis shortcuts, else polar form
__device__ inline double2 csqrt_nc(double2 z) {
  if (z.y == 0.0) {
    if (!signbit(z.x)) return make_double2(sqrt(z.x), z.y);
    double im = sqrt(-z.x);
    return signbit(z.y) ? make_double2(0.0, -im) : make_double2(0.0, im);
  }
  if (z.x == 0.0) {
    double x = sqrt(fabs(z.y) / 2.0);
    return signbit(z.y) ? make_double2(x, -x) : make_double2(x, x);
  }
  double r = hypot(z.x, z.y);
  double th = atan2(z.y, z.x) / 2.0;
  double rs = sqrt(r);
  return make_double2(rs * cos(th), rs * sin(th));
}
// Complex::tanh: (sinh 2a + i sin 2b) / (cosh 2a + cos 2b)
__device__ inline double2 ctanh_nc(double2 z) {
  double a2 = z.x + z.x, b2 = z.y + z.y;
  double den = cosh(a2) + cos(b2);
  return make_double2(sinh(a2) / den, sin(b2) / den);
}
// gelu_complex (utils/activation.rs:195-212); powi(3) = z * (z * z)
__device__ inline double2 gelu_nc(double2 z, bool* nan) {
  const double s = 0x1.9884533d43651p-1;  // (2.0 / PI).sqrt() as f64 (correctly rounded sqrt)
  double2 z3 = cmul(z, cmul(z, z));
  double2 f = cscale(cadd(z, cmul(make_double2(0.044715, 0.0), z3)), s);
  double2 cl = make_double2(fmin(fmax(f.x, -30.0), 30.0), fmin(fmax(f.y, -30.0), 30.0));
  double2 t = ctanh_nc(cl);
  if (isnan(t.x) || isnan(t.y)) *nan = true;
  return cmul(cscale(z, 0.5), make_double2(1.0 + t.x, 0.0 + t.y));
}

// ---- wavefront reductions (wave64) ----
// ---- cross-lane reductions without the LDS crossbar ----
// DPP moves inside rows of 16 lanes (quad swaps, half-row and row mirrors,
// row rotate by 8) and gfx950's v_permlane16_swap / v_permlane32_swap across
// rows take a few cycles each, where ds_bpermute (what __shfl_xor becomes)
// is an LDS round trip.  Every step combines a lane with a partner that
// combines the same two operands (mirrors pair uniform groups once the quads
// are reduced; a swap hands both rows the same pair), so all lanes of a
// group end with the same bits.
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1, 0, 3, 2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2, 3, 0, 1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane j of 8 <- 7 - j
constexpr int DPP_MIRROR = 0x140;      // lane j of 16 <- 15 - j
constexpr int DPP_ROR8 = 0x128;        // lane j of 16 <- (j + 8) % 16, i.e. j ^ 8

template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true); }
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  return __hiloint2double(dpp_i32<CTRL>(__double2hiint(v)), dpp_i32<CTRL>(__double2loint(v)));
}
// a: the even 16-lane row of the lane's row pair, b: the odd one (same in both rows)
__device__ __forceinline__ void pair16_f64(double v, double& a, double& b) {
  const auto lo = __builtin_amdgcn_permlane16_swap((unsigned)__double2loint(v), (unsigned)__double2loint(v), false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap((unsigned)__double2hiint(v), (unsigned)__double2hiint(v), false, false);
  a = __hiloint2double((int)hi[0], (int)lo[0]);
  b = __hiloint2double((int)hi[1], (int)lo[1]);
}
// a: lanes 0-31, b: lanes 32-63 (same in both halves)
__device__ __forceinline__ void pair32_f64(double v, double& a, double& b) {
  const auto lo = __builtin_amdgcn_permlane32_swap((unsigned)__double2loint(v), (unsigned)__double2loint(v), false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap((unsigned)__double2hiint(v), (unsigned)__double2hiint(v), false, false);
  a = __hiloint2double((int)hi[0], (int)lo[0]);
  b = __hiloint2double((int)hi[1], (int)lo[1]);
}
__device__ __forceinline__ void pair16_i32(int v, int& a, int& b) {
  const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  a = (int)r[0];
  b = (int)r[1];
}
__device__ __forceinline__ void pair32_i32(int v, int& a, int& b) {
  const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  a = (int)r[0];
  b = (int)r[1];
}

// sum / max over each row of 16 lanes
__device__ __forceinline__ double row16_sum(double v) {
  v += dpp_f64<DPP_XOR1>(v);
  v += dpp_f64<DPP_XOR2>(v);
  v += dpp_f64<DPP_HALF_MIRROR>(v);
  v += dpp_f64<DPP_MIRROR>(v);
  return v;
}
__device__ __forceinline__ double row16_max(double v) {
  v = fmax(v, dpp_f64<DPP_XOR1>(v));
  v = fmax(v, dpp_f64<DPP_XOR2>(v));
  v = fmax(v, dpp_f64<DPP_HALF_MIRROR>(v));
  v = fmax(v, dpp_f64<DPP_MIRROR>(v));
  return v;
}
// sums over lanes j, j ^ 16, j ^ 32, j ^ 48 (xor16), j ^ 32 (xor32), j ^ 8 (xor8)
__device__ __forceinline__ double xor16_sum(double v) {
  double a, b;
  pair16_f64(v, a, b);
  return a + b;
}
__device__ __forceinline__ double xor32_sum(double v) {
  double a, b;
  pair32_f64(v, a, b);
  return a + b;
}
__device__ __forceinline__ double xor8_sum(double v) { return v + dpp_f64<DPP_ROR8>(v); }
// sum of the lanes sharing lane % C (C in 8, 16, 32, 64)
template <int C>
__device__ __forceinline__ double col_sum(double v) {
  if constexpr (C <= 8) v = xor8_sum(v);
  if constexpr (C <= 16) v = xor16_sum(v);
  if constexpr (C <= 32) v = xor32_sum(v);
  return v;
}
__device__ __forceinline__ double wave_sum(double v) { return xor32_sum(xor16_sum(row16_sum(v))); }
__device__ __forceinline__ double wave_max(double v) {
  v = row16_max(v);
  double a, b;
  pair16_f64(v, a, b);
  v = fmax(a, b);
  pair32_f64(v, a, b);
  return fmax(a, b);
}

// ---- cross-block results (split partials) ----
// MI355X has one L2 per XCD and they are not coherent with each other, so the
// partial results one block leaves for another (split-K, key chunks, argmax
// tiles) are written and read at device coherence (relaxed agent-scope
// atomics: the sc1 stores/loads that reach past the XCD's L2).  An
// agent-scope fence would instead write back and invalidate the whole L2,
// which measured several times slower than the whole product.
// Every pointer is cast to the global address space: a pointer the compiler
// cannot trace to a kernel argument (one read from a table in memory, as the
// resident loop's operations are) would otherwise become a FLAT access, which
// also counts against lgkmcnt, so each later LDS or scalar wait would wait for
// every load in flight.
#define MITOK_GLOBAL __attribute__((address_space(1)))
__device__ __forceinline__ void st_dev(double* p, double v) {
  __hip_atomic_store((MITOK_GLOBAL unsigned long long*)p, (unsigned long long)__double_as_longlong(v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double ld_dev(const double* p) {
  return __longlong_as_double((long long)__hip_atomic_load((MITOK_GLOBAL unsigned long long*)p, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st_dev(double2* p, double2 v) {
  st_dev(&p->x, v.x);
  st_dev(&p->y, v.y);
}
__device__ __forceinline__ double2 ld_dev(const double2* p) { return make_double2(ld_dev(&p->x), ld_dev(&p->y)); }
__device__ __forceinline__ void st_dev(int* p, int v) {
  __hip_atomic_store((MITOK_GLOBAL int*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_dev(const int* p) {
  return __hip_atomic_load((MITOK_GLOBAL int*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store((MITOK_GLOBAL uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
  return __hip_atomic_load((MITOK_GLOBAL uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// an ordinary load of data nothing writes during the kernel (weights, tables)
template <class T>
__device__ __forceinline__ T ld_glb(const T* p) {
  return *(const MITOK_GLOBAL T*)p;
}
// double2's copy constructor takes a generic reference, so it is loaded as a
// plain vector
__device__ __forceinline__ double2 ld_glb(const double2* p) {
  const v2d v = *(const MITOK_GLOBAL v2d*)p;
  return make_double2(v.x, v.y);
}
// a streamed weight: read once per pass, so the load is non-temporal and the
// caches keep the activations, flags and code instead
__device__ __forceinline__ double2 ld_stream(const double2* p) {
  const v2d v = __builtin_nontemporal_load((const MITOK_GLOBAL v2d*)p);
  return make_double2(v.x, v.y);
}

// Access policy of the shared device code (rowops.hpp, epilogue.hpp) for
// data that may change while a kernel runs.  AccPlain: ordinary loads and
// stores, for kernels that only read what earlier launches wrote.  The
// resident decode loop (resident.hip), where every block runs until the last
// step, supplies a policy with device-coherent activations and the per-step
// state (KV lengths, ids, history count) kept in each block's LDS.
//   ld / st    activations and partial results
//   c          weights and tables (nothing writes them during a launch)
//   kv(p, m)   KV length of sequence m (also the RoPE position of its new token)
//   id(p, m)   token id of row m
//   cnt(p)     decode-step count (the logits-history slot)
struct AccPlain {
  template <class T>
  static __device__ __forceinline__ T ld(const T* p) { return *p; }
  template <class T>
  static __device__ __forceinline__ void st(T* p, T v) { *p = v; }
  template <class T>
  static __device__ __forceinline__ T c(const T* p) { return *p; }
  static __device__ __forceinline__ int kv(const int* p, int m) { return p[m]; }
  static __device__ __forceinline__ uint32_t id(const uint32_t* p, int m) { return p[m]; }
  static __device__ __forceinline__ int cnt(const int* p) { return p[0]; }
};

// ---- split completion ----
// Every block of a split calls this once after writing its partial result
// with st_dev; it returns true in exactly one block, the last to arrive, which
// then reads every partial with ld_dev.  Each wave first waits for its stores
// to be acknowledged (vmcnt counts stores on gfx9), so they are device-visible
// before the counter moves.  The counter is reset by the last block, so the
// next launch on the stream starts from zero.  All threads of the block must
// call it (it contains barriers).
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expected) {
  __shared__ uint32_t s_last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    MITOK_GLOBAL uint32_t* c = (MITOK_GLOBAL uint32_t*)counter;
    const uint32_t old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = (old + 1u == expected) ? 1u : 0u;
    if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  return s_last != 0u;
}

// greedy_decoding order: the larger value wins, equal values go to the larger
// index (Rust max_by keeps the last maximum); index -1 marks "no value"
__device__ __forceinline__ void argmax_combine(double& bv, int& bi, double ov, int oi) {
  if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
    bv = ov;
    bi = oi;
  }
}
// the combine is symmetric (larger value, then larger index), so partners agree
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(double& v, int& i) {
  argmax_combine(v, i, dpp_f64<CTRL>(v), dpp_i32<CTRL>(i));
}
__device__ __forceinline__ void row16_argmax(double& v, int& i) {
  argmax_dpp<DPP_XOR1>(v, i);
  argmax_dpp<DPP_XOR2>(v, i);
  argmax_dpp<DPP_HALF_MIRROR>(v, i);
  argmax_dpp<DPP_MIRROR>(v, i);
}
__device__ __forceinline__ void wave_argmax(double& v, int& i) {
  row16_argmax(v, i);
  double a, b;
  int ia, ib;
  pair16_f64(v, a, b);
  pair16_i32(i, ia, ib);
  argmax_combine(a, ia, b, ib);
  pair32_f64(a, v, b);
  pair32_i32(ia, i, ib);
  argmax_combine(v, i, b, ib);
}

}  // namespace mitok
