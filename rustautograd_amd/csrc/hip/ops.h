// Device semantics of rg's elementwise operations, shared by the precompiled kernels and the
// source of every JIT-compiled fused group. The text between RG_OPS_BEGIN/RG_OPS_END is both
// compiled here and kept as a string (rg_ops_source) for hiprtc, so the two paths cannot drift.
//
// Semantics follow the reference's CPU interpreter (src/plan.rs:972-995, 1190-1210,
// src/tensor.rs:215-227): NaN-propagating max/min, sign(+-0) = +-0, comparisons give 0/1 in the
// operand dtype, `where` selects on c != 0, transcendental functions per element with no fast
// math and no contraction.
#pragma once

#define RG_STRINGIZE_(...) #__VA_ARGS__
#define RG_DEFINE_OPS(...) \
  __VA_ARGS__              \
  static const char* const rg_ops_source = RG_STRINGIZE_(__VA_ARGS__);

RG_DEFINE_OPS(
  __device__ __forceinline__ float rg_exp(float x) { return expf(x); }
  __device__ __forceinline__ double rg_exp(double x) { return exp(x); }
  __device__ __forceinline__ float rg_log(float x) { return logf(x); }
  __device__ __forceinline__ double rg_log(double x) { return log(x); }
  __device__ __forceinline__ float rg_sqrt(float x) { return sqrtf(x); }
  __device__ __forceinline__ double rg_sqrt(double x) { return sqrt(x); }
  __device__ __forceinline__ float rg_sin(float x) { return sinf(x); }
  __device__ __forceinline__ double rg_sin(double x) { return sin(x); }
  __device__ __forceinline__ float rg_cos(float x) { return cosf(x); }
  __device__ __forceinline__ double rg_cos(double x) { return cos(x); }
  __device__ __forceinline__ float rg_tanh(float x) { return tanhf(x); }
  __device__ __forceinline__ double rg_tanh(double x) { return tanh(x); }
  __device__ __forceinline__ float rg_abs(float x) { return fabsf(x); }
  __device__ __forceinline__ double rg_abs(double x) { return fabs(x); }
  __device__ __forceinline__ float rg_floor(float x) { return floorf(x); }
  __device__ __forceinline__ double rg_floor(double x) { return floor(x); }
  __device__ __forceinline__ float rg_pow(float x, float y) { return powf(x, y); }
  __device__ __forceinline__ double rg_pow(double x, double y) { return pow(x, y); }
  template <class T> __device__ __forceinline__ T rg_sign(T x) { return x > (T)0 ? (T)1 : (x < (T)0 ? (T)-1 : x); }
  template <class T> __device__ __forceinline__ T rg_max(T a, T b) { return a > b ? a : (b >= a ? b : (T)__builtin_nan("")); }
  template <class T> __device__ __forceinline__ T rg_min(T a, T b) { return a < b ? a : (b <= a ? b : (T)__builtin_nan("")); }
  template <class T> __device__ __forceinline__ T rg_gt(T a, T b) { return a > b ? (T)1 : (T)0; }
  template <class T> __device__ __forceinline__ T rg_ge(T a, T b) { return a >= b ? (T)1 : (T)0; }
  template <class T> __device__ __forceinline__ T rg_where(T c, T a, T b) { return c != (T)0 ? a : b; }
  // Wave64 all-reductions without LDS: within each row of 16 lanes by DPP (quad exchanges, then
  // the half-row and row mirrors), then across rows with the permlane swaps. Every lane combines
  // the same two values at every step, so every lane ends with the same bits.
  template <int C> __device__ __forceinline__ float rg_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), C, 0xf, 0xf, false));
  }
  template <int C> __device__ __forceinline__ double rg_dpp(double x) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(x);
    const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)b, C, 0xf, 0xf, false);
    const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), C, 0xf, 0xf, false);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
  }
  __device__ __forceinline__ void rg_swap16(float x, float* a, float* b) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    *a = __uint_as_float(p[0]);
    *b = __uint_as_float(p[1]);
  }
  __device__ __forceinline__ void rg_swap32(float x, float* a, float* b) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    *a = __uint_as_float(p[0]);
    *b = __uint_as_float(p[1]);
  }
  __device__ __forceinline__ void rg_swap16(double x, double* a, double* b) {
    const unsigned long long v = (unsigned long long)__double_as_longlong(x);
    const auto lo = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((unsigned)(v >> 32), (unsigned)(v >> 32), false, false);
    *a = __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0]));
    *b = __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
  }
  __device__ __forceinline__ void rg_swap32(double x, double* a, double* b) {
    const unsigned long long v = (unsigned long long)__double_as_longlong(x);
    const auto lo = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((unsigned)(v >> 32), (unsigned)(v >> 32), false, false);
    *a = __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0]));
    *b = __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
  }
  template <class T, class F> __device__ __forceinline__ T rg_wave_all(T x, F f) {
    x = f(x, rg_dpp<0xB1>(x));   /* quad_perm [1,0,3,2] */
    x = f(x, rg_dpp<0x4E>(x));   /* quad_perm [2,3,0,1] */
    x = f(x, rg_dpp<0x141>(x));  /* row_half_mirror */
    x = f(x, rg_dpp<0x140>(x));  /* row_mirror */
    T a, b;
    rg_swap16(x, &a, &b);
    x = f(a, b);
    rg_swap32(x, &a, &b);
    return f(a, b);
  }
  template <class T> __device__ __forceinline__ T rg_wave_sum(T x) { return rg_wave_all(x, [](T a, T b) { return a + b; }); }
  template <class T> __device__ __forceinline__ T rg_wave_max(T x) { return rg_wave_all(x, [](T a, T b) { return rg_max(a, b); }); }
  template <class T> __device__ __forceinline__ T rg_wave_min(T x) { return rg_wave_all(x, [](T a, T b) { return rg_min(a, b); }); }
)

// Opcode dispatch for the precompiled single-operation kernels (RG_OP_* of rg_plan.h).
template <class T>
__device__ __forceinline__ T rg_unary(int op, T x) {
  switch (op) {
    case RG_OP_NEG: return -x;
    case RG_OP_EXP: return rg_exp(x);
    case RG_OP_LOG: return rg_log(x);
    case RG_OP_SQRT: return rg_sqrt(x);
    case RG_OP_SIN: return rg_sin(x);
    case RG_OP_COS: return rg_cos(x);
    case RG_OP_TANH: return rg_tanh(x);
    case RG_OP_ABS: return rg_abs(x);
    case RG_OP_SIGN: return rg_sign(x);
    case RG_OP_FLOOR: return rg_floor(x);
    default: return x;
  }
}

template <class T>
__device__ __forceinline__ T rg_binary(int op, T a, T b) {
  switch (op) {
    case RG_OP_ADD: return a + b;
    case RG_OP_SUB: return a - b;
    case RG_OP_MUL: return a * b;
    case RG_OP_DIV: return a / b;
    case RG_OP_POW: return rg_pow(a, b);
    case RG_OP_MAX: return rg_max(a, b);
    case RG_OP_MIN: return rg_min(a, b);
    case RG_OP_GT: return rg_gt(a, b);
    case RG_OP_GE: return rg_ge(a, b);
    default: return a;
  }
}

// int32 arithmetic wraps (src/plan.rs:1272-1287).
__device__ __forceinline__ int rg_binary_int(int op, int a, int b) {
  switch (op) {
    case RG_OP_ADD: return (int)((unsigned)a + (unsigned)b);
    case RG_OP_SUB: return (int)((unsigned)a - (unsigned)b);
    case RG_OP_MUL: return (int)((unsigned)a * (unsigned)b);
    case RG_OP_GT: return a > b;
    case RG_OP_GE: return a >= b;
    default: return a;
  }
}
