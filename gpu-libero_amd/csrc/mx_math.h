// Device math helpers for the world-local step kernel (gfx950).
// Quaternions are w,x,y,z; spatial vectors are [angular; linear] (MuJoCo's convention, used by the
// reference's leaves, e.g. gpu/cuda/dynamics/mjwarp_spatial.cuh).
#pragma once
#include <hip/hip_runtime.h>

// The step is compiled with each world's working set in LDS (namespace mx, the default) and, for
// models whose working set exceeds the LDS of a workgroup, in a per-world slab of device memory
// (namespaces mx_slab and mx_slab4, MX_SLAB defined; address space 1 = global).  The physics
// working type `real` is float; the FP64 build (namespace mx_f64, MX_F64 defined, LDS working set
// only) makes it double.  The model image stays 32-bit words in every build.
#ifndef MX_NS
#define MX_NS mx
#endif
#ifdef MX_SLAB
#define MX_WS_AS 1
#else
#define MX_WS_AS 3
#endif

namespace MX_NS {

// Working-set pointer types (LDS in the default build).  Structures that hold pointers into the
// working set keep this address space so that functions the compiler does not inline still emit
// LDS (or global) instructions: a generic pointer loaded from memory would be accessed through the
// slower flat path.
#ifdef MX_F64
#ifdef MX_SLAB
#error "the FP64 build keeps its working set in LDS"
#endif
typedef double real;
#else
typedef float real;
#endif
constexpr int kRealWords = (int)(sizeof(real) / 4);   // 32-bit working-set words per real
typedef __attribute__((address_space(MX_WS_AS))) float lfloat;
typedef __attribute__((address_space(MX_WS_AS))) real lreal;
typedef __attribute__((address_space(MX_WS_AS))) int lint;
typedef __attribute__((address_space(MX_WS_AS))) double ldouble;
typedef __attribute__((address_space(MX_WS_AS))) unsigned long long lu64;
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(MX_WS_AS))) v4f lfloat4;
typedef __attribute__((address_space(3))) double sdouble;   // always LDS
typedef __attribute__((address_space(3))) float sfloat;
typedef __attribute__((address_space(3))) real sreal;
typedef __attribute__((address_space(3))) int sint;
typedef __attribute__((address_space(3))) short sshort;   // LDS copies of small indices
typedef __attribute__((address_space(3))) unsigned long long su64;
typedef __attribute__((address_space(3))) v4f sfloat4;

// ---- math of the working type: each helper has a float and a double form (the float forms are the
// single-precision library calls)
__device__ __forceinline__ float r_sqrt(float x) { return sqrtf(x); }
__device__ __forceinline__ double r_sqrt(double x) { return sqrt(x); }
__device__ __forceinline__ float r_rsqrt(float x) { return rsqrtf(x); }
__device__ __forceinline__ double r_rsqrt(double x) { return rsqrt(x); }
__device__ __forceinline__ float r_abs(float x) { return fabsf(x); }
__device__ __forceinline__ double r_abs(double x) { return fabs(x); }
__device__ __forceinline__ float r_max(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ double r_max(double a, double b) { return fmax(a, b); }
__device__ __forceinline__ float r_min(float a, float b) { return fminf(a, b); }
__device__ __forceinline__ double r_min(double a, double b) { return fmin(a, b); }
// mixed float and double arguments (a model constant beside a working value) take the double form
__device__ __forceinline__ double r_max(double a, float b) { return fmax(a, (double)b); }
__device__ __forceinline__ double r_max(float a, double b) { return fmax((double)a, b); }
__device__ __forceinline__ double r_min(double a, float b) { return fmin(a, (double)b); }
__device__ __forceinline__ double r_min(float a, double b) { return fmin((double)a, b); }
__device__ __forceinline__ void r_sincos(float x, float* s, float* c) { sincosf(x, s, c); }
__device__ __forceinline__ void r_sincos(double x, double* s, double* c) { sincos(x, s, c); }
__device__ __forceinline__ float r_exp(float x) { return expf(x); }
__device__ __forceinline__ double r_exp(double x) { return exp(x); }
__device__ __forceinline__ float r_log(float x) { return logf(x); }
__device__ __forceinline__ double r_log(double x) { return log(x); }
__device__ __forceinline__ float r_pow(float x, float y) { return powf(x, y); }
__device__ __forceinline__ double r_pow(double x, double y) { return pow(x, y); }
__device__ __forceinline__ double r_pow(double x, float y) { return pow(x, (double)y); }
__device__ __forceinline__ double r_pow(float x, double y) { return pow((double)x, y); }
__device__ __forceinline__ float r_atan2(float y, float x) { return atan2f(y, x); }
__device__ __forceinline__ double r_atan2(double y, double x) { return atan2(y, x); }
__device__ __forceinline__ float r_acos(float x) { return acosf(x); }
__device__ __forceinline__ double r_acos(double x) { return acos(x); }
__device__ __forceinline__ float r_floor(float x) { return floorf(x); }
__device__ __forceinline__ double r_floor(double x) { return floor(x); }
__device__ __forceinline__ float r_copysign(float x, float y) { return copysignf(x, y); }
__device__ __forceinline__ double r_copysign(double x, double y) { return copysign(x, y); }
__device__ __forceinline__ float r_tan(float x) { return tanf(x); }
__device__ __forceinline__ double r_tan(double x) { return tan(x); }
__device__ __forceinline__ float r_atan(float x) { return atanf(x); }
__device__ __forceinline__ double r_atan(double x) { return atan(x); }
__device__ __forceinline__ float r_sin(float x) { return sinf(x); }
__device__ __forceinline__ double r_sin(double x) { return sin(x); }
__device__ __forceinline__ float r_cos(float x) { return cosf(x); }
__device__ __forceinline__ double r_cos(double x) { return cos(x); }

// ---- wave-wide reductions and scans with DPP (data-parallel primitives move values between lanes
// inside the VALU: quad permutes, row shifts, mirrors and the row broadcasts 15 and 31).  A lane
// that a row mask or an out-of-row source leaves unwritten reads the operation's identity, so each
// step is `v = op(v, moved)`; a reduction collects in lane 63 and is read back wave-uniform.
template <int kCtrl, int kRowMask, int kBankMask = 0xF>
__device__ __forceinline__ int dpp_move(int identity, int v) {
  return __builtin_amdgcn_update_dpp(identity, v, kCtrl, kRowMask, kBankMask, false);
}
template <class Op>
__device__ __forceinline__ int dpp_reduce(int v, int identity, Op op) {
  v = op(v, dpp_move<0xB1, 0xF>(identity, v));    // quad_perm [1,0,3,2]
  v = op(v, dpp_move<0x4E, 0xF>(identity, v));    // quad_perm [2,3,0,1]
  v = op(v, dpp_move<0x141, 0xF>(identity, v));   // row_half_mirror
  v = op(v, dpp_move<0x140, 0xF>(identity, v));   // row_mirror
  v = op(v, dpp_move<0x142, 0xA>(identity, v));   // row_bcast:15 into rows 1, 3
  v = op(v, dpp_move<0x143, 0xC>(identity, v));   // row_bcast:31 into rows 2, 3
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ float wave_sum(float v) {
  return __int_as_float(dpp_reduce(__float_as_int(v), 0, [](int a, int b) {
    return __float_as_int(__int_as_float(a) + __int_as_float(b));
  }));
}
__device__ __forceinline__ float wave_min(float v) {
  return __int_as_float(dpp_reduce(__float_as_int(v), __float_as_int(__builtin_inff()), [](int a, int b) {
    return __float_as_int(fminf(__int_as_float(a), __int_as_float(b)));
  }));
}
__device__ __forceinline__ float wave_max(float v) {
  return __int_as_float(dpp_reduce(__float_as_int(v), __float_as_int(-__builtin_inff()), [](int a, int b) {
    return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b)));
  }));
}
__device__ __forceinline__ int wave_min(int v) {
  return dpp_reduce(v, 0x7fffffff, [](int a, int b) { return a < b ? a : b; });
}
// the same over each row of 16 lanes: after the quad permutes and the two mirrors every lane of a
// row holds the row's result (no broadcast needed)
template <class Op>
__device__ __forceinline__ int dpp_row_reduce(int v, int identity, Op op) {
  v = op(v, dpp_move<0xB1, 0xF>(identity, v));    // quad_perm [1,0,3,2]
  v = op(v, dpp_move<0x4E, 0xF>(identity, v));    // quad_perm [2,3,0,1]
  v = op(v, dpp_move<0x141, 0xF>(identity, v));   // row_half_mirror
  v = op(v, dpp_move<0x140, 0xF>(identity, v));   // row_mirror
  return v;
}
__device__ __forceinline__ float row_min(float v) {
  return __int_as_float(dpp_row_reduce(__float_as_int(v), __float_as_int(__builtin_inff()), [](int a, int b) {
    return __float_as_int(fminf(__int_as_float(a), __int_as_float(b)));
  }));
}
__device__ __forceinline__ float row_max(float v) {
  return __int_as_float(dpp_row_reduce(__float_as_int(v), __float_as_int(-__builtin_inff()), [](int a, int b) {
    return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b)));
  }));
}
__device__ __forceinline__ int row_min(int v) {
  return dpp_row_reduce(v, 0x7fffffff, [](int a, int b) { return a < b ? a : b; });
}
// the double forms: both 32-bit halves move with the same DPP control
template <int kCtrl, int kRowMask, int kBankMask = 0xF>
__device__ __forceinline__ double dpp_move(double identity, double v) {
  const long long i = __double_as_longlong(identity), x = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp((int)i, (int)x, kCtrl, kRowMask, kBankMask, false);
  const int hi = __builtin_amdgcn_update_dpp((int)(i >> 32), (int)(x >> 32), kCtrl, kRowMask, kBankMask, false);
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
__device__ __forceinline__ float read_lane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ int read_lane(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ double read_lane(double v, int lane) {
  const long long x = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)x, lane), hi = __builtin_amdgcn_readlane((int)(x >> 32), lane);
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
template <class Op>
__device__ __forceinline__ double dpp_reduce(double v, double identity, Op op) {
  v = op(v, dpp_move<0xB1, 0xF>(identity, v));
  v = op(v, dpp_move<0x4E, 0xF>(identity, v));
  v = op(v, dpp_move<0x141, 0xF>(identity, v));
  v = op(v, dpp_move<0x140, 0xF>(identity, v));
  v = op(v, dpp_move<0x142, 0xA>(identity, v));
  v = op(v, dpp_move<0x143, 0xC>(identity, v));
  return read_lane(v, 63);
}
template <class Op>
__device__ __forceinline__ double dpp_row_reduce(double v, double identity, Op op) {
  v = op(v, dpp_move<0xB1, 0xF>(identity, v));
  v = op(v, dpp_move<0x4E, 0xF>(identity, v));
  v = op(v, dpp_move<0x141, 0xF>(identity, v));
  v = op(v, dpp_move<0x140, 0xF>(identity, v));
  return v;
}
__device__ __forceinline__ double wave_sum(double v) {
  return dpp_reduce(v, 0.0, [](double a, double b) { return a + b; });
}
__device__ __forceinline__ double wave_min(double v) {
  return dpp_reduce(v, __builtin_inf(), [](double a, double b) { return fmin(a, b); });
}
__device__ __forceinline__ double wave_max(double v) {
  return dpp_reduce(v, -__builtin_inf(), [](double a, double b) { return fmax(a, b); });
}
__device__ __forceinline__ double row_min(double v) {
  return dpp_row_reduce(v, __builtin_inf(), [](double a, double b) { return fmin(a, b); });
}
__device__ __forceinline__ double row_max(double v) {
  return dpp_row_reduce(v, -__builtin_inf(), [](double a, double b) { return fmax(a, b); });
}

// inclusive prefix sum over the 64 lanes (lane order)
__device__ __forceinline__ int wave_incl_scan(int v) {
  int x = v;
  x += dpp_move<0x111, 0xF>(0, v);         // row_shr:1
  x += dpp_move<0x112, 0xF>(0, v);         // row_shr:2
  x += dpp_move<0x113, 0xF>(0, v);         // row_shr:3: x = v[l-3..l] within the row
  x += dpp_move<0x114, 0xF, 0xE>(0, x);    // row_shr:4 into lanes 4-15 of each row
  x += dpp_move<0x118, 0xF, 0xC>(0, x);    // row_shr:8 into lanes 8-15: prefix within the row
  x += dpp_move<0x142, 0xA>(0, x);         // row_bcast:15: rows 1, 3 add the previous row's total
  x += dpp_move<0x143, 0xC>(0, x);         // row_bcast:31: rows 2, 3 add the total of rows 0-1
  return x;
}

__device__ __forceinline__ void qmul(const real* a, const real* b, real* r) {
  real w = a[0] * b[0] - a[1] * b[1] - a[2] * b[2] - a[3] * b[3];
  real x = a[0] * b[1] + a[1] * b[0] + a[2] * b[3] - a[3] * b[2];
  real y = a[0] * b[2] - a[1] * b[3] + a[2] * b[0] + a[3] * b[1];
  real z = a[0] * b[3] + a[1] * b[2] - a[2] * b[1] + a[3] * b[0];
  r[0] = w; r[1] = x; r[2] = y; r[3] = z;
}

__device__ __forceinline__ void quat2mat(const real* q, real* r) {
  real q00 = q[0] * q[0], q01 = q[0] * q[1], q02 = q[0] * q[2], q03 = q[0] * q[3];
  real q11 = q[1] * q[1], q12 = q[1] * q[2], q13 = q[1] * q[3];
  real q22 = q[2] * q[2], q23 = q[2] * q[3], q33 = q[3] * q[3];
  r[0] = q00 + q11 - q22 - q33; r[4] = q00 - q11 + q22 - q33; r[8] = q00 - q11 - q22 + q33;
  r[1] = 2.f * (q12 - q03); r[2] = 2.f * (q13 + q02); r[3] = 2.f * (q12 + q03);
  r[5] = 2.f * (q23 - q01); r[6] = 2.f * (q13 - q02); r[7] = 2.f * (q23 + q01);
}

__device__ __forceinline__ void normalize4(real* q) {
  real n = r_sqrt(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
  if (n < 1e-15f) { q[0] = 1.f; q[1] = q[2] = q[3] = 0.f; return; }
  real inv = 1.f / n;
  q[0] *= inv; q[1] *= inv; q[2] *= inv; q[3] *= inv;
}

__device__ __forceinline__ void mulmv3(const real* m, const real* v, real* r) {
  real a = m[0] * v[0] + m[1] * v[1] + m[2] * v[2];
  real b = m[3] * v[0] + m[4] * v[1] + m[5] * v[2];
  real c = m[6] * v[0] + m[7] * v[1] + m[8] * v[2];
  r[0] = a; r[1] = b; r[2] = c;
}

__device__ __forceinline__ void mulmm3(const real* a, const real* b, real* r) {
  real t[9];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) t[3 * i + j] = a[3 * i] * b[j] + a[3 * i + 1] * b[3 + j] + a[3 * i + 2] * b[6 + j];
#pragma unroll
  for (int k = 0; k < 9; ++k) r[k] = t[k];
}

__device__ __forceinline__ void cross3(const real* a, const real* b, real* r) {
  real x = a[1] * b[2] - a[2] * b[1], y = a[2] * b[0] - a[0] * b[2], z = a[0] * b[1] - a[1] * b[0];
  r[0] = x; r[1] = y; r[2] = z;
}

__device__ __forceinline__ void mul_inert_vec(const real* i, const real* v, real* r) {
  real r0 = i[0] * v[0] + i[3] * v[1] + i[4] * v[2] - i[8] * v[4] + i[7] * v[5];
  real r1 = i[3] * v[0] + i[1] * v[1] + i[5] * v[2] + i[8] * v[3] - i[6] * v[5];
  real r2 = i[4] * v[0] + i[5] * v[1] + i[2] * v[2] - i[7] * v[3] + i[6] * v[4];
  real r3 = i[8] * v[1] - i[7] * v[2] + i[9] * v[3];
  real r4 = i[6] * v[2] - i[8] * v[0] + i[9] * v[4];
  real r5 = i[7] * v[0] - i[6] * v[1] + i[9] * v[5];
  r[0] = r0; r[1] = r1; r[2] = r2; r[3] = r3; r[4] = r4; r[5] = r5;
}

__device__ __forceinline__ void cross_motion(const real* v, const real* u, real* r) {
  r[0] = -v[2] * u[1] + v[1] * u[2];
  r[1] = v[2] * u[0] - v[0] * u[2];
  r[2] = -v[1] * u[0] + v[0] * u[1];
  r[3] = -v[2] * u[4] + v[1] * u[5] - v[5] * u[1] + v[4] * u[2];
  r[4] = v[2] * u[3] - v[0] * u[5] + v[5] * u[0] - v[3] * u[2];
  r[5] = -v[1] * u[3] + v[0] * u[4] - v[4] * u[0] + v[3] * u[1];
}

__device__ __forceinline__ void cross_force(const real* v, const real* f, real* r) {
  r[0] = -v[2] * f[1] + v[1] * f[2] - v[5] * f[4] + v[4] * f[5];
  r[1] = v[2] * f[0] - v[0] * f[2] + v[5] * f[3] - v[3] * f[5];
  r[2] = -v[1] * f[0] + v[0] * f[1] - v[4] * f[3] + v[3] * f[4];
  r[3] = -v[2] * f[4] + v[1] * f[5];
  r[4] = v[2] * f[3] - v[0] * f[5];
  r[5] = -v[1] * f[3] + v[0] * f[4];
}

#ifdef MX_F64
// FP32 model-image operands of the FP64 build, widened to the working type first
__device__ __forceinline__ void quat2mat(const float* q, real* r) {
  const real t[4] = {q[0], q[1], q[2], q[3]};
  quat2mat(t, r);
}
__device__ __forceinline__ void mulmv3(const real* m, const float* v, real* r) {
  const real t[3] = {v[0], v[1], v[2]};
  mulmv3(m, t, r);
}
__device__ __forceinline__ void mulmv3(const float* m, const real* v, real* r) {
  real t[9];
  for (int k = 0; k < 9; ++k) t[k] = m[k];
  mulmv3(t, v, r);
}
__device__ __forceinline__ void mulmm3(const real* a, const float* b, real* r) {
  real t[9];
  for (int k = 0; k < 9; ++k) t[k] = b[k];
  mulmm3(a, t, r);
}
__device__ __forceinline__ void cross3(const float* a, const real* b, real* r) {
  const real t[3] = {a[0], a[1], a[2]};
  cross3(t, b, r);
}
__device__ __forceinline__ void cross3(const real* a, const float* b, real* r) {
  const real t[3] = {b[0], b[1], b[2]};
  cross3(a, t, r);
}
__device__ __forceinline__ void qmul(const real* a, const float* b, real* r) {
  const real t[4] = {b[0], b[1], b[2], b[3]};
  qmul(a, t, r);
}
#endif

}  // namespace mx
