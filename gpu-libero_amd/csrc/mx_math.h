// Device math helpers for the world-local step kernel (gfx950).
// Quaternions are w,x,y,z; spatial vectors are [angular; linear] (MuJoCo's convention, used by the
// reference's leaves, e.g. gpu/cuda/dynamics/mjwarp_spatial.cuh).
#pragma once
#include <hip/hip_runtime.h>

// The step is compiled twice: with each world's working set in LDS (namespace mx, the default)
// and, for models whose working set exceeds the LDS of a workgroup, in a per-world slab of device
// memory (namespace mx_slab, MX_SLAB defined; address space 1 = global).
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
typedef __attribute__((address_space(MX_WS_AS))) float lfloat;
typedef __attribute__((address_space(MX_WS_AS))) int lint;
typedef __attribute__((address_space(MX_WS_AS))) double ldouble;
typedef __attribute__((address_space(MX_WS_AS))) unsigned long long lu64;
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(MX_WS_AS))) v4f lfloat4;
typedef __attribute__((address_space(3))) double sdouble;   // always LDS
typedef __attribute__((address_space(3))) float sfloat;
typedef __attribute__((address_space(3))) int sint;
typedef __attribute__((address_space(3))) unsigned long long su64;
typedef __attribute__((address_space(3))) v4f sfloat4;

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

__device__ __forceinline__ void qmul(const float* a, const float* b, float* r) {
  float w = a[0] * b[0] - a[1] * b[1] - a[2] * b[2] - a[3] * b[3];
  float x = a[0] * b[1] + a[1] * b[0] + a[2] * b[3] - a[3] * b[2];
  float y = a[0] * b[2] - a[1] * b[3] + a[2] * b[0] + a[3] * b[1];
  float z = a[0] * b[3] + a[1] * b[2] - a[2] * b[1] + a[3] * b[0];
  r[0] = w; r[1] = x; r[2] = y; r[3] = z;
}

__device__ __forceinline__ void quat2mat(const float* q, float* r) {
  float q00 = q[0] * q[0], q01 = q[0] * q[1], q02 = q[0] * q[2], q03 = q[0] * q[3];
  float q11 = q[1] * q[1], q12 = q[1] * q[2], q13 = q[1] * q[3];
  float q22 = q[2] * q[2], q23 = q[2] * q[3], q33 = q[3] * q[3];
  r[0] = q00 + q11 - q22 - q33; r[4] = q00 - q11 + q22 - q33; r[8] = q00 - q11 - q22 + q33;
  r[1] = 2.f * (q12 - q03); r[2] = 2.f * (q13 + q02); r[3] = 2.f * (q12 + q03);
  r[5] = 2.f * (q23 - q01); r[6] = 2.f * (q13 - q02); r[7] = 2.f * (q23 + q01);
}

__device__ __forceinline__ void normalize4(float* q) {
  float n = sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
  if (n < 1e-15f) { q[0] = 1.f; q[1] = q[2] = q[3] = 0.f; return; }
  float inv = 1.f / n;
  q[0] *= inv; q[1] *= inv; q[2] *= inv; q[3] *= inv;
}

__device__ __forceinline__ void mulmv3(const float* m, const float* v, float* r) {
  float a = m[0] * v[0] + m[1] * v[1] + m[2] * v[2];
  float b = m[3] * v[0] + m[4] * v[1] + m[5] * v[2];
  float c = m[6] * v[0] + m[7] * v[1] + m[8] * v[2];
  r[0] = a; r[1] = b; r[2] = c;
}

__device__ __forceinline__ void mulmm3(const float* a, const float* b, float* r) {
  float t[9];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) t[3 * i + j] = a[3 * i] * b[j] + a[3 * i + 1] * b[3 + j] + a[3 * i + 2] * b[6 + j];
#pragma unroll
  for (int k = 0; k < 9; ++k) r[k] = t[k];
}

__device__ __forceinline__ void cross3(const float* a, const float* b, float* r) {
  float x = a[1] * b[2] - a[2] * b[1], y = a[2] * b[0] - a[0] * b[2], z = a[0] * b[1] - a[1] * b[0];
  r[0] = x; r[1] = y; r[2] = z;
}

__device__ __forceinline__ void mul_inert_vec(const float* i, const float* v, float* r) {
  float r0 = i[0] * v[0] + i[3] * v[1] + i[4] * v[2] - i[8] * v[4] + i[7] * v[5];
  float r1 = i[3] * v[0] + i[1] * v[1] + i[5] * v[2] + i[8] * v[3] - i[6] * v[5];
  float r2 = i[4] * v[0] + i[5] * v[1] + i[2] * v[2] - i[7] * v[3] + i[6] * v[4];
  float r3 = i[8] * v[1] - i[7] * v[2] + i[9] * v[3];
  float r4 = i[6] * v[2] - i[8] * v[0] + i[9] * v[4];
  float r5 = i[7] * v[0] - i[6] * v[1] + i[9] * v[5];
  r[0] = r0; r[1] = r1; r[2] = r2; r[3] = r3; r[4] = r4; r[5] = r5;
}

__device__ __forceinline__ void cross_motion(const float* v, const float* u, float* r) {
  r[0] = -v[2] * u[1] + v[1] * u[2];
  r[1] = v[2] * u[0] - v[0] * u[2];
  r[2] = -v[1] * u[0] + v[0] * u[1];
  r[3] = -v[2] * u[4] + v[1] * u[5] - v[5] * u[1] + v[4] * u[2];
  r[4] = v[2] * u[3] - v[0] * u[5] + v[5] * u[0] - v[3] * u[2];
  r[5] = -v[1] * u[3] + v[0] * u[4] - v[4] * u[0] + v[3] * u[1];
}

__device__ __forceinline__ void cross_force(const float* v, const float* f, float* r) {
  r[0] = -v[2] * f[1] + v[1] * f[2] - v[5] * f[4] + v[4] * f[5];
  r[1] = v[2] * f[0] - v[0] * f[2] + v[5] * f[3] - v[3] * f[5];
  r[2] = -v[1] * f[0] + v[0] * f[1] - v[4] * f[3] + v[3] * f[4];
  r[3] = -v[2] * f[4] + v[1] * f[5];
  r[4] = v[2] * f[3] - v[0] * f[5];
  r[5] = -v[1] * f[3] + v[0] * f[4];
}

}  // namespace mx
