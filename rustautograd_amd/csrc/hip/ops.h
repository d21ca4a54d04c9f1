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
