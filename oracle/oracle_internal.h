// Internal declarations of the CPU FP64 oracle -- TEST INFRASTRUCTURE ONLY (see oracle.h).
#pragma once
#include "oracle.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <vector>

namespace orc {

typedef double T;
constexpr T kMinVal = 1e-15;   // MuJoCo mjMINVAL

// ------------------------------------------------------------------ small vector algebra
inline void qmul(const T* a, const T* b, T* r) {
  T w = a[0] * b[0] - a[1] * b[1] - a[2] * b[2] - a[3] * b[3];
  T x = a[0] * b[1] + a[1] * b[0] + a[2] * b[3] - a[3] * b[2];
  T y = a[0] * b[2] - a[1] * b[3] + a[2] * b[0] + a[3] * b[1];
  T z = a[0] * b[3] + a[1] * b[2] - a[2] * b[1] + a[3] * b[0];
  r[0] = w; r[1] = x; r[2] = y; r[3] = z;
}
inline void quat2mat(const T* q, T* r) {
  T q00 = q[0] * q[0], q01 = q[0] * q[1], q02 = q[0] * q[2], q03 = q[0] * q[3];
  T q11 = q[1] * q[1], q12 = q[1] * q[2], q13 = q[1] * q[3];
  T q22 = q[2] * q[2], q23 = q[2] * q[3], q33 = q[3] * q[3];
  r[0] = q00 + q11 - q22 - q33; r[4] = q00 - q11 + q22 - q33; r[8] = q00 - q11 - q22 + q33;
  r[1] = 2 * (q12 - q03); r[2] = 2 * (q13 + q02); r[3] = 2 * (q12 + q03);
  r[5] = 2 * (q23 - q01); r[6] = 2 * (q13 - q02); r[7] = 2 * (q23 + q01);
}
inline void normalize4(T* q) {
  T n = std::sqrt(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
  if (n < kMinVal) { q[0] = 1; q[1] = q[2] = q[3] = 0; return; }
  for (int i = 0; i < 4; ++i) q[i] /= n;
}
inline void mulmv3(const T* m, const T* v, T* r) {
  T a = m[0] * v[0] + m[1] * v[1] + m[2] * v[2];
  T b = m[3] * v[0] + m[4] * v[1] + m[5] * v[2];
  T c = m[6] * v[0] + m[7] * v[1] + m[8] * v[2];
  r[0] = a; r[1] = b; r[2] = c;
}
inline void mulmtv3(const T* m, const T* v, T* r) {   // m^T v
  T a = m[0] * v[0] + m[3] * v[1] + m[6] * v[2];
  T b = m[1] * v[0] + m[4] * v[1] + m[7] * v[2];
  T c = m[2] * v[0] + m[5] * v[1] + m[8] * v[2];
  r[0] = a; r[1] = b; r[2] = c;
}
inline void mulmm3(const T* a, const T* b, T* r) {
  T t[9];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) t[3 * i + j] = a[3 * i] * b[j] + a[3 * i + 1] * b[3 + j] + a[3 * i + 2] * b[6 + j];
  std::memcpy(r, t, sizeof t);
}
inline void cross(const T* a, const T* b, T* r) {
  T x = a[1] * b[2] - a[2] * b[1], y = a[2] * b[0] - a[0] * b[2], z = a[0] * b[1] - a[1] * b[0];
  r[0] = x; r[1] = y; r[2] = z;
}
inline T dot3(const T* a, const T* b) { return a[0] * b[0] + a[1] * b[1] + a[2] * b[2]; }
inline T norm3(const T* a) { return std::sqrt(dot3(a, a)); }

// ------------------------------------------------------------------ contacts and rows
struct Contact {
  T pos[3], frame[9], dist, friction[5], solref[2], solimp[5], includemargin;
  int geom[2], dim, efc_address;
};

struct World {
  std::vector<T> xpos, xquat, xmat, xipos, ximat, xanchor, xaxis, subtree_com, cinert, crb;
  std::vector<T> cdof, cvel, cdof_dot, cacc, cfrc, M, L, L2, geom_xpos, geom_xmat, site_xpos, site_xmat;
  std::vector<T> qfrc_bias, qfrc_passive, qfrc_actuator, qfrc_smooth, qacc_smooth, qacc, qfrc_constraint;
  std::vector<T> actuator_force, jacp, jacr, tmp;
  // gravity compensation and applied body wrenches projected on the dofs; post-constraint outputs
  std::vector<T> qfrc_gravcomp, qfrc_xfrc, cfrc_ext, cacc_post, cfrc_int;
  // contacts and constraint rows
  std::vector<Contact> contacts;
  int ne = 0, nf = 0, nl = 0, nefc = 0, overflow = 0, niter = 0;
  std::vector<T> J;                      // nefc x nv dense
  std::vector<T> D, aref, efc_pos, efc_vel, frictionloss, force, jaref, jv, quad;
  std::vector<int> type, id, state;
  // Newton workspace
  std::vector<T> Ma, grad, search, Mv, H, Hf;
  explicit World(const OrModel& m);
};

// stages (oracle.cpp)
void kinematics(const OrModel& m, const T* qpos, World& w);
void com_pos(const OrModel& m, World& w);
void crb(const OrModel& m, World& w);
void factor(const OrModel& m, const T* M, T* L, const T* diag_add, T scale);
void solve(const OrModel& m, const T* L, T* x);
void mul_m(const OrModel& m, const T* M, const T* x, T* y);
void body_jac(const OrModel& m, const World& w, int body, const T* point, T* jacp, T* jacr);

// collision (oracle_collision.cpp): fills w.contacts from the current frames
void collision(const OrModel& m, World& w, const int32_t* body_active);

// constraint rows and the Newton solver (oracle_solver.cpp)
void make_constraint(const OrModel& m, World& w, const T* qpos, const T* qvel);
void newton(const OrModel& m, World& w, const T* warmstart);

}  // namespace orc
