// World-local control-step kernel for gfx950 (MI355X) and the C ABI of libmx_physics.so.
//
// One 64-lane wavefront owns one world for a whole control step: the world's state and every
// intermediate (frames, cinert, cdof, mass blocks and factors, bias forces, controller matrices)
// live in LDS, and the `substeps` physics substeps run inside one launch.  Each substep follows the
// reference schedule step1 -> OSC -> solve -> integrate (gpu/host/backends/cuda_fp32/runtime.py:40-45,
// physics.py:585-633); the stages and their reference leaves are named at each device function.
// HBM is touched only to load the state at entry and to publish state and derived fields at exit.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstring>
#include <cmath>
#include "../../include/mx_physics.h"
#include "mx_math.h"

namespace mx {

constexpr int kLanes = 64;

// Offsets of the per-world LDS arena.  Floats first (offsets in floats), then doubles (offsets in
// doubles from `dbase`, a byte offset aligned to 8).
struct Layout {
  int qpos, qvel, ctrl, warm, applied, xpos, xquat, xmat, xipos, ximat, xanchor, xaxis, scom, cinert, crb;
  int cdof, cvel, cdofdot, cfrcb, cfrc, M, L, gxpos, gxmat, sxpos, sxmat, bias, passive, act, smooth;
  int qacc_smooth, qacc, qcon, tmp, actforce, jacp, jacr, misc, nfloat;
  int dbase;
  int m7, minv, J, mjt, A, Ap, Ar, Lf, Lp, Lr, jbar, N, q, qd, dbias, eepos, eerot, eevel;
  int goalpos, goalrot, grip, R, desired, wrench, pd, posture, tau, dctrl, work, ndouble;
  int bytes;
};

inline int round_up(int x, int a) { return (x + a - 1) / a * a; }

Layout make_layout(const MxModel& m) {
  Layout L{};
  int at = 0;
  auto take = [&](int n) { int o = at; at += round_up(n > 0 ? n : 1, 4); return o; };
  int nb = m.nbody, nv = m.nv, nj = m.njnt;
  L.qpos = take(m.nq); L.qvel = take(nv); L.ctrl = take(m.nu); L.warm = take(nv); L.applied = take(nv);
  L.xpos = take(3 * nb); L.xquat = take(4 * nb); L.xmat = take(9 * nb); L.xipos = take(3 * nb);
  L.ximat = take(9 * nb); L.xanchor = take(3 * nj); L.xaxis = take(3 * nj); L.scom = take(3 * nb);
  L.cinert = take(10 * nb); L.crb = take(10 * nb); L.cdof = take(6 * nv); L.cvel = take(6 * nb);
  L.cdofdot = take(6 * nv); L.cfrcb = take(6 * nb); L.cfrc = take(6 * nb); L.M = take(m.nM); L.L = take(m.nM);
  L.gxpos = take(3 * m.ngeom); L.gxmat = take(9 * m.ngeom); L.sxpos = take(3 * m.nsite); L.sxmat = take(9 * m.nsite);
  L.bias = take(nv); L.passive = take(nv); L.act = take(nv); L.smooth = take(nv); L.qacc_smooth = take(nv);
  L.qacc = take(nv); L.qcon = take(nv); L.tmp = take(nv); L.actforce = take(m.nu);
  L.jacp = take(3 * 7); L.jacr = take(3 * 7); L.misc = take(16);
  L.nfloat = at;
  L.dbase = round_up(at * 4, 16);
  int dt = 0;
  auto dtake = [&](int n) { int o = dt; dt += round_up(n, 2); return o; };
  L.m7 = dtake(49); L.minv = dtake(49); L.J = dtake(42); L.mjt = dtake(42); L.A = dtake(36);
  L.Ap = dtake(9); L.Ar = dtake(9); L.Lf = dtake(36); L.Lp = dtake(9); L.Lr = dtake(9);
  L.jbar = dtake(42); L.N = dtake(49); L.q = dtake(7); L.qd = dtake(7); L.dbias = dtake(7);
  L.eepos = dtake(3); L.eerot = dtake(9); L.eevel = dtake(6); L.goalpos = dtake(3); L.goalrot = dtake(9);
  L.grip = dtake(2); L.R = dtake(9); L.desired = dtake(6); L.wrench = dtake(6); L.pd = dtake(7);
  L.posture = dtake(7); L.tau = dtake(7); L.dctrl = dtake(9); L.work = dtake(3 * 72 + 8);
  L.ndouble = dt;
  L.bytes = L.dbase + dt * 8;
  return L;
}

// Scalars shared by the lanes of a world (in the `misc` LDS slot, as ints or floats).
enum Misc { kFail = 0, kCtrlErr = 1, kPinvFail = 2, kRank0 = 3 };

struct Ctx {
  const MxModel& m;
  const MxData& d;
  const Layout& L;
  float* f;      // LDS floats
  double* g;     // LDS doubles
  int w, lane;
  __device__ float* F(int off) const { return f + off; }
  __device__ double* D(int off) const { return g + off; }
};

__device__ __forceinline__ void sync() { __syncthreads(); }

// ---------------------------------------------------------------- position stage
// Forward kinematics, level by level (bodies of one tree depth in parallel lanes): MuJoCo
// mj_kinematics semantics; reference fused leaf gpu/cuda/fp32/fused_kinematic_mass.cu:110-447.
__device__ void kinematics(const Ctx& c) {
  const MxModel& m = c.m;
  float *xpos = c.F(c.L.xpos), *xquat = c.F(c.L.xquat), *xmat = c.F(c.L.xmat);
  const float* qpos = c.F(c.L.qpos);
  if (c.lane == 0) {
    xpos[0] = xpos[1] = xpos[2] = 0.f;
    xquat[0] = 1.f; xquat[1] = xquat[2] = xquat[3] = 0.f;
    for (int k = 0; k < 9; ++k) xmat[k] = (k % 4 == 0) ? 1.f : 0.f;
  }
  sync();
  for (int lv = 1; lv <= m.nlevel; ++lv) {
    int a = m.level_adr[lv - 1], e = m.level_adr[lv];
    for (int k = a + c.lane; k < e; k += kLanes) {
      int b = m.level_body[k], p = m.body_parent[b];
      float pos[3], quat[4], off[3];
      mulmv3(xmat + 9 * p, m.body_pos + 3 * b, off);
      for (int i = 0; i < 3; ++i) pos[i] = xpos[3 * p + i] + off[i];
      qmul(xquat + 4 * p, m.body_quat + 4 * b, quat);
      for (int j = m.body_jntadr[b]; j < m.body_jntadr[b] + m.body_jntnum[b]; ++j) {
        int qa = m.jnt_qposadr[j], type = m.jnt_type[j];
        float* anc = c.F(c.L.xanchor) + 3 * j;
        float* ax = c.F(c.L.xaxis) + 3 * j;
        if (type == 0) {
          for (int i = 0; i < 3; ++i) pos[i] = qpos[qa + i];
          for (int i = 0; i < 4; ++i) quat[i] = qpos[qa + 3 + i];
          normalize4(quat);
          for (int i = 0; i < 3; ++i) anc[i] = pos[i];
          ax[0] = 0.f; ax[1] = 0.f; ax[2] = 1.f;
          continue;
        }
        float R[9], an[3], axis[3];
        quat2mat(quat, R);
        mulmv3(R, m.jnt_pos + 3 * j, an);
        for (int i = 0; i < 3; ++i) an[i] += pos[i];
        mulmv3(R, m.jnt_axis + 3 * j, axis);
        for (int i = 0; i < 3; ++i) { anc[i] = an[i]; ax[i] = axis[i]; }
        float delta = qpos[qa] - m.qpos0[qa];
        if (type == 2) {
          for (int i = 0; i < 3; ++i) pos[i] += axis[i] * delta;
        } else if (type == 3) {
          float s, co;
          sincosf(0.5f * delta, &s, &co);
          float ql[4] = {co, m.jnt_axis[3 * j] * s, m.jnt_axis[3 * j + 1] * s, m.jnt_axis[3 * j + 2] * s};
          float nq[4];
          qmul(quat, ql, nq);
          for (int i = 0; i < 4; ++i) quat[i] = nq[i];
          quat2mat(quat, R);
          float r[3];
          mulmv3(R, m.jnt_pos + 3 * j, r);
          for (int i = 0; i < 3; ++i) pos[i] = an[i] - r[i];
        }
      }
      normalize4(quat);
      for (int i = 0; i < 3; ++i) xpos[3 * b + i] = pos[i];
      for (int i = 0; i < 4; ++i) xquat[4 * b + i] = quat[i];
      quat2mat(quat, xmat + 9 * b);
    }
    sync();
  }
  // inertial, geom and site frames (independent per object)
  for (int b = c.lane; b < m.nbody; b += kLanes) {
    float off[3], R[9];
    mulmv3(xmat + 9 * b, m.body_ipos + 3 * b, off);
    for (int i = 0; i < 3; ++i) c.F(c.L.xipos)[3 * b + i] = xpos[3 * b + i] + off[i];
    quat2mat(m.body_iquat + 4 * b, R);
    mulmm3(xmat + 9 * b, R, c.F(c.L.ximat) + 9 * b);
  }
  for (int g = c.lane; g < m.ngeom; g += kLanes) {
    int b = m.geom_body[g];
    float off[3], R[9];
    mulmv3(xmat + 9 * b, m.geom_pos + 3 * g, off);
    for (int i = 0; i < 3; ++i) c.F(c.L.gxpos)[3 * g + i] = xpos[3 * b + i] + off[i];
    quat2mat(m.geom_quat + 4 * g, R);
    mulmm3(xmat + 9 * b, R, c.F(c.L.gxmat) + 9 * g);
  }
  for (int s = c.lane; s < m.nsite; s += kLanes) {
    int b = m.site_body[s];
    float off[3], R[9];
    mulmv3(xmat + 9 * b, m.site_pos + 3 * s, off);
    for (int i = 0; i < 3; ++i) c.F(c.L.sxpos)[3 * s + i] = xpos[3 * b + i] + off[i];
    quat2mat(m.site_quat + 4 * s, R);
    mulmm3(xmat + 9 * b, R, c.F(c.L.sxmat) + 9 * s);
  }
  sync();
}

// Subtree com (contiguous DFS subtree sums), cinert and cdof: MuJoCo mj_comPos; reference
// gpu/cuda/dynamics/mjwarp_com_pos.cu:95 and fused_kinematic_mass.cu (centered frames).
__device__ void com_pos(const Ctx& c) {
  const MxModel& m = c.m;
  const float* xipos = c.F(c.L.xipos);
  float* scom = c.F(c.L.scom);
  for (int b = c.lane; b < m.nbody; b += kLanes) {
    float s[3] = {0.f, 0.f, 0.f};
    int e = b + m.body_subtreesize[b];
    for (int k = b; k < e; ++k) {
      float mk = m.body_mass[k];
      for (int i = 0; i < 3; ++i) s[i] += mk * xipos[3 * k + i];
    }
    float sm = m.body_subtreemass[b];
    for (int i = 0; i < 3; ++i) scom[3 * b + i] = sm < 1e-15f ? xipos[3 * b + i] : s[i] / sm;
  }
  sync();
  for (int b = c.lane; b < m.nbody; b += kLanes) {
    float* ci = c.F(c.L.cinert) + 10 * b;
    if (b == 0) { for (int k = 0; k < 10; ++k) ci[k] = 0.f; continue; }
    const float* R = c.F(c.L.ximat) + 9 * b;
    const float* I = m.body_inertia + 3 * b;
    float mass = m.body_mass[b], dd[3];
    int r = m.body_rootid[b];
    for (int i = 0; i < 3; ++i) dd[i] = xipos[3 * b + i] - scom[3 * r + i];
    float rot[9];
    for (int i = 0; i < 3; ++i)
      for (int j = 0; j < 3; ++j)
        rot[3 * i + j] = R[3 * i] * I[0] * R[3 * j] + R[3 * i + 1] * I[1] * R[3 * j + 1] + R[3 * i + 2] * I[2] * R[3 * j + 2];
    ci[0] = rot[0] + mass * (dd[1] * dd[1] + dd[2] * dd[2]);
    ci[1] = rot[4] + mass * (dd[0] * dd[0] + dd[2] * dd[2]);
    ci[2] = rot[8] + mass * (dd[0] * dd[0] + dd[1] * dd[1]);
    ci[3] = rot[1] - mass * dd[0] * dd[1];
    ci[4] = rot[2] - mass * dd[0] * dd[2];
    ci[5] = rot[5] - mass * dd[1] * dd[2];
    ci[6] = mass * dd[0]; ci[7] = mass * dd[1]; ci[8] = mass * dd[2]; ci[9] = mass;
  }
  for (int j = c.lane; j < m.njnt; j += kLanes) {
    int b = m.jnt_body[j], da = m.jnt_dofadr[j], r = m.body_rootid[b];
    const float* anc = c.F(c.L.xanchor) + 3 * j;
    const float* ax = c.F(c.L.xaxis) + 3 * j;
    float off[3];
    for (int i = 0; i < 3; ++i) off[i] = scom[3 * r + i] - anc[i];
    float* cd = c.F(c.L.cdof);
    int type = m.jnt_type[j];
    if (type == 0) {
      for (int dd = 0; dd < 3; ++dd) {
        float* o = cd + 6 * (da + dd);
        for (int k = 0; k < 6; ++k) o[k] = 0.f;
        o[3 + dd] = 1.f;
      }
      const float* X = c.F(c.L.xmat) + 9 * b;
      for (int dd = 0; dd < 3; ++dd) {
        float* o = cd + 6 * (da + 3 + dd);
        float a3[3] = {X[dd], X[3 + dd], X[6 + dd]};
        o[0] = a3[0]; o[1] = a3[1]; o[2] = a3[2];
        cross3(a3, off, o + 3);
      }
    } else if (type == 2) {
      float* o = cd + 6 * da;
      o[0] = o[1] = o[2] = 0.f; o[3] = ax[0]; o[4] = ax[1]; o[5] = ax[2];
    } else if (type == 3) {
      float* o = cd + 6 * da;
      o[0] = ax[0]; o[1] = ax[1]; o[2] = ax[2];
      cross3(ax, off, o + 3);
    }
  }
  sync();
}

// Composite inertia (subtree sums) and the dense per-tree mass blocks from (dof, ancestor dof)
// pairs: MuJoCo mj_crb; reference fused_kinematic_mass.cu (CRB, CSR M) / mjwarp_mass_matrix.cu:54.
__device__ void crb_mass(const Ctx& c) {
  const MxModel& m = c.m;
  const float* ci = c.F(c.L.cinert);
  float* crb = c.F(c.L.crb);
  float* M = c.F(c.L.M);
  for (int t = c.lane; t < 10 * m.nbody; t += kLanes) {
    int b = t / 10, k = t % 10;
    float s = 0.f;
    if (b > 0) {
      int e = b + m.body_subtreesize[b];
      for (int q = b; q < e; ++q) s += ci[10 * q + k];
    }
    crb[t] = s;
  }
  for (int t = c.lane; t < m.nM; t += kLanes) M[t] = 0.f;
  sync();
  const float* cdof = c.F(c.L.cdof);
  for (int p = c.lane; p < m.nMpair; p += kLanes) {
    int i = m.mpair_i[p], j = m.mpair_j[p];
    float buf[6];
    mul_inert_vec(crb + 10 * m.dof_body[i], cdof + 6 * i, buf);
    float v = 0.f;
    for (int k = 0; k < 6; ++k) v += cdof[6 * j + k] * buf[k];
    if (i == j) v += m.dof_armature[i];
    int t = m.dof_treeid[i], n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    float* blk = M + m.tree_madr[t];
    blk[(i - a) * n + (j - a)] = v;
    blk[(j - a) * n + (i - a)] = v;
  }
  sync();
}

// Per-tree dense Cholesky (one lane per tree): reference gpu/cuda/dynamics/mjwarp_mass_factor.cu:134-247.
__device__ void factor(const Ctx& c, const float* M, float* Lf, const float* diag_add, float scale) {
  const MxModel& m = c.m;
  for (int t = c.lane; t < m.ntree; t += kLanes) {
    int n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    const float* A = M + m.tree_madr[t];
    float* F = Lf + m.tree_madr[t];
    for (int j = 0; j < n; ++j) {
      float dj = A[j * n + j] + (diag_add ? scale * diag_add[a + j] : 0.f);
      for (int k = 0; k < j; ++k) dj -= F[j * n + k] * F[j * n + k];
      dj = sqrtf(fmaxf(dj, 1e-15f));
      F[j * n + j] = dj;
      float inv = 1.f / dj;
      for (int i = j + 1; i < n; ++i) {
        float v = A[i * n + j];
        for (int k = 0; k < j; ++k) v -= F[i * n + k] * F[j * n + k];
        F[i * n + j] = v * inv;
      }
    }
  }
  sync();
}

// x <- M^-1 x per tree with the factor (POTRS role, gpu/cuda/dynamics/mjwarp_mass_solve.cu:74-122).
__device__ void solve(const Ctx& c, const float* Lf, float* x) {
  const MxModel& m = c.m;
  for (int t = c.lane; t < m.ntree; t += kLanes) {
    int n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    const float* F = Lf + m.tree_madr[t];
    float* v = x + a;
    for (int i = 0; i < n; ++i) {
      float s = v[i];
      for (int k = 0; k < i; ++k) s -= F[i * n + k] * v[k];
      v[i] = s / F[i * n + i];
    }
    for (int i = n - 1; i >= 0; --i) {
      float s = v[i];
      for (int k = i + 1; k < n; ++k) s -= F[k * n + i] * v[k];
      v[i] = s / F[i * n + i];
    }
  }
  sync();
}

// ---------------------------------------------------------------- velocity stage
// cvel, cdof_dot, RNE bias forces and passive forces: MuJoCo mj_comVel + mj_rne(0) + mj_passive;
// reference gpu/cuda/fp32/fused_motion_passive.cu:43-387 / fused_motion.cu:14 / mjwarp_passive.cu.
__device__ void velocity(const Ctx& c) {
  const MxModel& m = c.m;
  const float* qvel = c.F(c.L.qvel);
  const float* cdof = c.F(c.L.cdof);
  float* cvel = c.F(c.L.cvel);
  float* cdd = c.F(c.L.cdofdot);
  for (int b = c.lane; b < m.nbody; b += kLanes) {
    float v[6] = {0, 0, 0, 0, 0, 0};
    for (int dd = m.body_lastdof[b]; dd >= 0; dd = m.dof_parent[dd])
      for (int k = 0; k < 6; ++k) v[k] += cdof[6 * dd + k] * qvel[dd];
    for (int k = 0; k < 6; ++k) cvel[6 * b + k] = v[k];
  }
  for (int i = c.lane; i < m.nv; i += kLanes) {
    int j = m.dof_jnt[i], da = m.jnt_dofadr[j];
    float v[6] = {0, 0, 0, 0, 0, 0};
    int start;
    if (m.jnt_type[j] == 0) start = i - da >= 3 ? da + 2 : -1;   // free: translations only
    else start = m.dof_parent[i];
    for (int dd = start; dd >= 0; dd = m.dof_parent[dd])
      for (int k = 0; k < 6; ++k) v[k] += cdof[6 * dd + k] * qvel[dd];
    cross_motion(v, cdof + 6 * i, cdd + 6 * i);
  }
  sync();
  const float* ci = c.F(c.L.cinert);
  float* cfb = c.F(c.L.cfrcb);
  float g[3] = {0.f, 0.f, 0.f};
  if (!(m.opt_disableflags & (1 << 6))) { g[0] = -m.opt_gravity_x; g[1] = -m.opt_gravity_y; g[2] = -m.opt_gravity_z; }
  for (int b = c.lane; b < m.nbody; b += kLanes) {
    if (b == 0) { for (int k = 0; k < 6; ++k) cfb[k] = 0.f; continue; }
    float a[6] = {0, 0, 0, g[0], g[1], g[2]};
    for (int dd = m.body_lastdof[b]; dd >= 0; dd = m.dof_parent[dd])
      for (int k = 0; k < 6; ++k) a[k] += cdd[6 * dd + k] * qvel[dd];
    float f1[6], h[6], f2[6];
    mul_inert_vec(ci + 10 * b, a, f1);
    mul_inert_vec(ci + 10 * b, cvel + 6 * b, h);
    cross_force(cvel + 6 * b, h, f2);
    for (int k = 0; k < 6; ++k) cfb[6 * b + k] = f1[k] + f2[k];
  }
  sync();
  float* cfrc = c.F(c.L.cfrc);
  for (int t = c.lane; t < 6 * m.nbody; t += kLanes) {
    int b = t / 6, k = t % 6;
    float s = 0.f;
    if (b > 0) {
      int e = b + m.body_subtreesize[b];
      for (int q = b; q < e; ++q) s += cfb[6 * q + k];
    }
    cfrc[t] = s;
  }
  sync();
  const float* qpos = c.F(c.L.qpos);
  for (int i = c.lane; i < m.nv; i += kLanes) {
    float s = 0.f;
    for (int k = 0; k < 6; ++k) s += cdof[6 * i + k] * cfrc[6 * m.dof_body[i] + k];
    c.F(c.L.bias)[i] = s;
    float p = 0.f;
    if (!(m.opt_disableflags & (1 << 5))) {
      int j = m.dof_jnt[i], type = m.jnt_type[j];
      if ((type == 2 || type == 3) && m.jnt_stiffness[j] != 0.f) {
        int qa = m.jnt_qposadr[j];
        p -= m.jnt_stiffness[j] * (qpos[qa] - m.qpos_spring[qa]);
      }
      p -= m.dof_damping[i] * qvel[i];
    }
    c.F(c.L.passive)[i] = p;
  }
  sync();
}

// ---------------------------------------------------------------- FP64 operational-space control
// Lane-parallel symmetric Gauss-Jordan inversion of up to three SPD operands at once (the OSC's
// M^-1, or A, A_pos, A_ori).  Lane `e` owns entry e of the concatenated problems.  Step k:
// row k <- (row k with a_kk := 1) / a_kk;  row i != k <- (row i with a_ik := 0) - a_ik * row k.
// A pivot that is not positive and finite marks the problem failed.
struct GJProblem { int base, n, first; };

__device__ void gj_inverse(const Ctx& c, const double* in, double* out, GJProblem p0, GJProblem p1,
                           GJProblem p2, int nprob, int* fail) {
  int lane = c.lane;
  int which = -1, n = 0, base = 0, e = 0;
  GJProblem ps[3] = {p0, p1, p2};
  for (int q = 0; q < nprob; ++q)
    if (lane >= ps[q].first && lane < ps[q].first + ps[q].n * ps[q].n) { which = q; n = ps[q].n; base = ps[q].base; e = lane - ps[q].first; }
  int i = which >= 0 ? e / n : 0, j = which >= 0 ? e % n : 0;
  double a = which >= 0 ? in[base + e] : 0.0;
  int bad = 0;
  int maxn = 0;
  for (int q = 0; q < nprob; ++q) maxn = ps[q].n > maxn ? ps[q].n : maxn;
  for (int k = 0; k < maxn; ++k) {
    if (which >= 0) out[base + e] = a;
    sync();
    if (which >= 0 && k < n) {
      double piv = out[base + k * n + k];
      if (!(piv > 0.0) || !isfinite(piv)) bad = 1;
      double rowk = (j == k ? 1.0 : out[base + k * n + j]) / piv;
      double colk = out[base + i * n + k];
      a = i == k ? rowk : (j == k ? 0.0 : a) - colk * rowk;
    }
    sync();
  }
  if (which >= 0) out[base + e] = a;
  for (int q = 0; q < nprob; ++q) fail[q] = 0;
  sync();
  if (which >= 0 && bad) atomicOr(&fail[which], 1);
  sync();
}

// Jacobi pseudo-inverse fallback for an operand whose inverse is not provably its pseudo-inverse
// (rank-deficient or worse than 1e13 conditioned); restates pinv_group
// (gpu/cuda/control/osc_solver.cu:108-258).  Serial in one lane; rare.
__device__ int jacobi_pinv(const double* a, int n, double* out, int* rank, double* B, double* V) {
  double scale = 0.0;
  for (int k = 0; k < n * n; ++k) scale = fmax(scale, fabs(a[k]));
  for (int k = 0; k < n * n; ++k) out[k] = 0.0;
  *rank = 0;
  if (!(scale > 0.0)) return 1;
  for (int cc = 0; cc < n; ++cc)
    for (int r = 0; r < n; ++r) { B[cc * n + r] = a[r * n + cc] / scale; V[cc * n + r] = r == cc ? 1.0 : 0.0; }
  bool converged = false;
  for (int sweep = 0; sweep < 64; ++sweep) {
    int rotations = 0;
    for (int p = 0; p < n - 1; ++p)
      for (int q = p + 1; q < n; ++q) {
        double alpha = 0, beta = 0, gamma = 0;
        for (int r = 0; r < n; ++r) {
          alpha += B[p * n + r] * B[p * n + r];
          beta += B[q * n + r] * B[q * n + r];
          gamma += B[p * n + r] * B[q * n + r];
        }
        if (fabs(gamma) > 2.220446049250313e-16 * sqrt(alpha) * sqrt(beta)) {
          double zeta = (beta - alpha) / (2 * gamma);
          double t = (zeta < 0 ? -1.0 : 1.0) / (fabs(zeta) + sqrt(1 + zeta * zeta));
          double cs = 1 / sqrt(1 + t * t), s = cs * t;
          for (int r = 0; r < n; ++r) {
            double bp = B[p * n + r], bq = B[q * n + r], vp = V[p * n + r], vq = V[q * n + r];
            B[p * n + r] = cs * bp - s * bq; B[q * n + r] = s * bp + cs * bq;
            V[p * n + r] = cs * vp - s * vq; V[q * n + r] = s * vp + cs * vq;
          }
          ++rotations;
        }
      }
    if (rotations == 0) { converged = true; break; }
  }
  double norms[6], sing[6], maxnorm = 0;
  bool keep[6];
  for (int p = 0; p < n; ++p) {
    double s = 0;
    for (int r = 0; r < n; ++r) s += B[p * n + r] * B[p * n + r];
    norms[p] = s; sing[p] = sqrt(s); maxnorm = fmax(maxnorm, sing[p]);
  }
  int count = 0;
  for (int p = 0; p < n; ++p) { keep[p] = sing[p] > 1e-15 * maxnorm; count += keep[p]; }
  double maxcorr = 0;
  for (int p = 0; p < n; ++p)
    for (int q = p + 1; q < n; ++q)
      if (keep[p] && keep[q]) {
        double gg = 0;
        for (int r = 0; r < n; ++r) gg += B[p * n + r] * B[q * n + r];
        maxcorr = fmax(maxcorr, fabs(gg) / (sing[p] * sing[q]));
      }
  if (maxcorr < 2e-15) converged = true;
  for (int r = 0; r < n; ++r)
    for (int cc = 0; cc < n; ++cc) {
      double v = 0;
      for (int k = 0; k < n; ++k)
        if (keep[k]) v += V[k * n + r] * B[k * n + cc] * ((1 / norms[k]) / scale);
      out[r * n + cc] = v;
    }
  *rank = count;
  return converged ? 1 : 0;
}

// robosuite's float32 quat2mat of an axis-angle delta (rotation_delta, osc_solver.cu:278-306);
// the float steps are kept unfused so that they round exactly as the CPU restatement does.
__device__ void rotation_delta(double x, double y, double z, double* r) {
#pragma clang fp contract(off)
  double angle = sqrt(x * x + y * y + z * z);
  if (angle == 0.0) {
    for (int k = 0; k < 9; ++k) r[k] = k % 4 == 0 ? 1.0 : 0.0;
    return;
  }
  double f = sin(angle * 0.5) / angle;
  float q[4] = {(float)cos(angle * 0.5), (float)(x * f), (float)(y * f), (float)(z * f)};
  float n = q[0] * q[0];
  n = n + q[1] * q[1];
  n = n + q[2] * q[2];
  n = n + q[3] * q[3];
  float s = (float)sqrt(2.0 / (double)n);
  float qs[4];
  for (int i = 0; i < 4; ++i) qs[i] = q[i] * s;
  float p11 = qs[1] * qs[1], p22 = qs[2] * qs[2], p33 = qs[3] * qs[3];
  float p12 = qs[1] * qs[2], p13 = qs[1] * qs[3], p23 = qs[2] * qs[3];
  float p01 = qs[0] * qs[1], p02 = qs[0] * qs[2], p03 = qs[0] * qs[3];
  r[0] = (1.0 - (double)p22) - (double)p33;
  r[4] = (1.0 - (double)p11) - (double)p33;
  r[8] = (1.0 - (double)p11) - (double)p22;
  r[1] = (double)(p12 - p03);
  r[2] = (double)(p13 + p02);
  r[3] = (double)(p12 + p03);
  r[5] = (double)(p23 - p01);
  r[6] = (double)(p13 - p02);
  r[7] = (double)(p23 + p01);
}

__device__ __forceinline__ double clip1(double v) { return isnan(v) ? v : fmin(1.0, fmax(-1.0, v)); }

// Controller gather (EE site Jacobian, 7x7 M, 6x7 J, q, qdot, bias, EE pose/velocity in FP32 as the
// reference's control_drive, gpu/cuda/fp32/fused_control_drive.cu:34-300) and the FP64 robosuite
// OSC_POSE (gpu/cuda/control/osc_solver.cu:309-678): M^-1, A = J M^-1 J^T, Lambda = pinv(A) (full,
// pos, ori), J-bar, nullspace N, goal update at the policy substep, uncoupled wrench, posture
// torque, clipping, gripper.  Writes ctrl[osc_actuator] in LDS.
__device__ void control(const Ctx& c, int policy, bool publish) {
  const MxModel& m = c.m;
  const MxData& d = c.d;
  const int w = c.w, lane = c.lane, nv = m.nv;
  int* misc = reinterpret_cast<int*>(c.F(c.L.misc));
  // EE site Jacobian for the 7 arm dofs and EE velocity over all dofs (FP32, as the reference)
  const float* cdof = c.F(c.L.cdof);
  const float* scom = c.F(c.L.scom);
  const float* qvel = c.F(c.L.qvel);
  int site = m.osc_site, sb = m.site_body[site], root = m.body_rootid[sb];
  float* jacp = c.F(c.L.jacp);
  float* jacr = c.F(c.L.jacr);
  const float* sp = c.F(c.L.sxpos) + 3 * site;
  if (lane < 7) {
    int di = m.osc_dofadr[lane];
    bool anc = false;
    for (int dd = m.body_lastdof[sb]; dd >= 0; dd = m.dof_parent[dd]) anc |= dd == di;
    float off[3] = {sp[0] - scom[3 * root], sp[1] - scom[3 * root + 1], sp[2] - scom[3 * root + 2]};
    float t[3];
    cross3(cdof + 6 * di, off, t);
    for (int k = 0; k < 3; ++k) {
      jacr[k * 7 + lane] = anc ? cdof[6 * di + k] : 0.f;
      jacp[k * 7 + lane] = anc ? cdof[6 * di + 3 + k] + t[k] : 0.f;
    }
  }
  double* gm = c.D(c.L.m7);
  double* gJ = c.D(c.L.J);
  if (lane < 49) {
    int i = lane / 7, j = lane % 7;
    int di = m.osc_dofadr[i], dj = m.osc_dofadr[j];
    int t = m.dof_treeid[di], n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    float v = m.dof_treeid[dj] == t ? c.F(c.L.M)[m.tree_madr[t] + (di - a) * n + (dj - a)] : 0.f;
    gm[lane] = v;
    if (publish) d.osc_mass[(size_t)49 * w + lane] = v;
  }
  sync();
  if (lane < 42) {
    int r = lane / 7, col = lane % 7;
    float v = r < 3 ? jacp[r * 7 + col] : jacr[(r - 3) * 7 + col];
    gJ[lane] = v;
    if (publish) d.osc_jac[(size_t)42 * w + lane] = v;
  }
  if (lane < 6) {
    // EE velocity: Jacobian over all dofs times qvel (only ancestors of the site contribute)
    float s = 0.f;
    for (int dd = m.body_lastdof[sb]; dd >= 0; dd = m.dof_parent[dd]) {
      float val;
      if (lane < 3) {
        float off[3] = {sp[0] - scom[3 * root], sp[1] - scom[3 * root + 1], sp[2] - scom[3 * root + 2]};
        float t[3];
        cross3(cdof + 6 * dd, off, t);
        val = cdof[6 * dd + 3 + lane] + t[lane];
      } else {
        val = cdof[6 * dd + lane - 3];
      }
      s += val * qvel[dd];
    }
    c.D(c.L.eevel)[lane] = s;
    if (publish) d.osc_ee_vel[(size_t)6 * w + lane] = s;
  }
  if (lane < 7) {
    int di = m.osc_dofadr[lane];
    float qv = c.F(c.L.qpos)[m.osc_qposadr[lane]], vv = qvel[di], bb = c.F(c.L.bias)[di];
    c.D(c.L.q)[lane] = qv; c.D(c.L.qd)[lane] = vv; c.D(c.L.dbias)[lane] = bb;
    if (publish) {
      d.osc_q[(size_t)7 * w + lane] = qv; d.osc_qvel[(size_t)7 * w + lane] = vv; d.osc_bias[(size_t)7 * w + lane] = bb;
    }
  }
  if (lane < 3) {
    float v = sp[lane];
    c.D(c.L.eepos)[lane] = v;
    if (publish) d.osc_ee_pos[(size_t)3 * w + lane] = v;
  }
  if (lane < 9) {
    float v = c.F(c.L.sxmat)[9 * site + lane];
    c.D(c.L.eerot)[lane] = v;
    if (publish) d.osc_ee_rot[(size_t)9 * w + lane] = v;
  }
  sync();
  if (misc[kCtrlErr] != 0) return;
  // M^-1 (7x7)
  int* sfail = misc + 8;
  gj_inverse(c, gm, c.D(c.L.minv), GJProblem{0, 7, 0}, GJProblem{0, 0, 64}, GJProblem{0, 0, 64}, 1, sfail);
  if (sfail[0]) {
    if (lane == 0) misc[kCtrlErr] = MX_OSC_SINGULAR_MASS;
    sync();
    return;
  }
  const double* minv = c.D(c.L.minv);
  double* mjt = c.D(c.L.mjt);
  if (lane < 42) {      // M^-1 J^T (7x6)
    int i = lane / 6, col = lane % 6;
    double s = 0;
    for (int k = 0; k < 7; ++k) s += minv[i * 7 + k] * gJ[col * 7 + k];
    mjt[lane] = s;
  }
  sync();
  double* A = c.D(c.L.A);
  if (lane < 36) {      // A = J M^-1 J^T
    int r = lane / 6, col = lane % 6;
    double s = 0;
    for (int k = 0; k < 7; ++k) s += gJ[r * 7 + k] * mjt[k * 6 + col];
    A[lane] = s;
    if (r < 3 && col < 3) c.D(c.L.Ap)[r * 3 + col] = s;
    if (r >= 3 && col >= 3) c.D(c.L.Ar)[(r - 3) * 3 + col - 3] = s;
  }
  sync();
  // A, A_pos, A_ori live contiguously (A then Ap then Ar); Lf, Lp, Lr likewise.
  gj_inverse(c, c.D(c.L.A), c.D(c.L.Lf), GJProblem{0, 6, 0}, GJProblem{c.L.Ap - c.L.A, 3, 36},
             GJProblem{c.L.Ar - c.L.A, 3, 45}, 3, sfail);
  if (lane < 3) {
    const double* src = lane == 0 ? c.D(c.L.A) : (lane == 1 ? c.D(c.L.Ap) : c.D(c.L.Ar));
    const double* inv = lane == 0 ? c.D(c.L.Lf) : (lane == 1 ? c.D(c.L.Lp) : c.D(c.L.Lr));
    int n = lane == 0 ? 6 : 3;
    bool fast = !sfail[lane];
    if (fast) {
      double ta = 0, ti = 0;
      for (int i = 0; i < n; ++i) { ta += src[i * n + i]; ti += inv[i * n + i]; }
      fast = ti > 0 && ta * ti <= 1e13;
    }
    misc[kRank0 + lane] = n;
    sfail[4 + lane] = fast ? 0 : 1;
  }
  sync();
  if (lane < 3 && sfail[4 + lane]) {
    const double* src = lane == 0 ? c.D(c.L.A) : (lane == 1 ? c.D(c.L.Ap) : c.D(c.L.Ar));
    double* inv = lane == 0 ? c.D(c.L.Lf) : (lane == 1 ? c.D(c.L.Lp) : c.D(c.L.Lr));
    int n = lane == 0 ? 6 : 3, rank = 0;
    double* work = c.D(c.L.work) + 72 * lane;
    int ok = jacobi_pinv(src, n, inv, &rank, work, work + 36);
    misc[kRank0 + lane] = rank;
    if (!ok) atomicOr(&misc[kPinvFail], 1);
  }
  sync();
  if (misc[kPinvFail]) {
    if (lane == 0) misc[kCtrlErr] = MX_OSC_PINV_FAILED;
    sync();
    return;
  }
  const double* Lf = c.D(c.L.Lf);
  double* jbar = c.D(c.L.jbar);
  if (lane < 42) {      // J-bar = M^-1 J^T Lambda (7x6)
    int i = lane / 6, col = lane % 6;
    double s = 0;
    for (int k = 0; k < 6; ++k) s += mjt[i * 6 + k] * Lf[k * 6 + col];
    jbar[lane] = s;
  }
  // goal update (policy substep): goal_pos = ee + 0.05 clip(a), goal_rot = R(0.5 clip(a)) ee_rot
  double* gp = c.D(c.L.goalpos);
  double* gr = c.D(c.L.goalrot);
  const double* eep = c.D(c.L.eepos);
  const double* eer = c.D(c.L.eerot);
  const double* action = d.osc_action + (size_t)7 * w;
  if (policy && lane == 0) {
    for (int k = 0; k < 3; ++k) gp[k] = eep[k] + 0.05 * clip1(action[k]);
    rotation_delta(0.5 * clip1(action[3]), 0.5 * clip1(action[4]), 0.5 * clip1(action[5]), c.D(c.L.R));
  }
  sync();
  if (policy && lane < 9) {
    const double* R = c.D(c.L.R);
    int i = lane / 3, j = lane % 3;
    gr[lane] = R[3 * i] * eer[j] + R[3 * i + 1] * eer[3 + j] + R[3 * i + 2] * eer[6 + j];
  }
  double* N = c.D(c.L.N);
  if (lane < 49) {      // N = I - J-bar J
    int i = lane / 7, j = lane % 7;
    double s = 0;
    for (int k = 0; k < 6; ++k) s += jbar[i * 6 + k] * gJ[k * 7 + j];
    N[lane] = (i == j ? 1.0 : 0.0) - s;
  }
  sync();
  const double* gains = d.osc_gains + (size_t)12 * w;
  const double* ev = c.D(c.L.eevel);
  double* desired = c.D(c.L.desired);
  double* pd = c.D(c.L.pd);
  if (lane < 3) {
    int r = lane, nx = (r + 1) % 3, ls = (r + 2) % 3;
    double er = 0;
    for (int cc = 0; cc < 3; ++cc) er += 0.5 * (eer[nx * 3 + cc] * gr[ls * 3 + cc] - eer[ls * 3 + cc] * gr[nx * 3 + cc]);
    double ep = gp[r] - eep[r];
    desired[r] = gains[r] * ep - gains[r + 6] * ev[r];
    desired[r + 3] = gains[r + 3] * er - gains[r + 9] * ev[r + 3];
  }
  if (lane >= 8 && lane < 15) {
    int cc = lane - 8;
    pd[cc] = 10.0 * (d.osc_q0[(size_t)7 * w + cc] - c.D(c.L.q)[cc]) - 6.324555320336759 * c.D(c.L.qd)[cc];
  }
  sync();
  double* wrench = c.D(c.L.wrench);
  double* posture = c.D(c.L.posture);
  if (lane < 6) {
    double s = 0;
    if (m.osc_uncouple) {
      const double* lam = lane < 3 ? c.D(c.L.Lp) : c.D(c.L.Lr);
      int r = lane % 3, o = lane < 3 ? 0 : 3;
      for (int k = 0; k < 3; ++k) s += lam[r * 3 + k] * desired[o + k];
    } else {
      for (int k = 0; k < 6; ++k) s += Lf[lane * 6 + k] * desired[k];
    }
    wrench[lane] = s;
  }
  if (lane >= 8 && lane < 15) {
    int r = lane - 8;
    double s = 0;
    for (int k = 0; k < 7; ++k) s += gm[r * 7 + k] * pd[k];
    posture[r] = s;
  }
  sync();
  float* ctrl = c.F(c.L.ctrl);
  if (lane < 7) {
    double task = 0, null = 0;
    for (int k = 0; k < 6; ++k) task += gJ[k * 7 + lane] * wrench[k];
    for (int k = 0; k < 7; ++k) null += N[k * 7 + lane] * posture[k];
    double t = task + c.D(c.L.dbias)[lane] + null;
    c.D(c.L.tau)[lane] = t;
    int act = m.osc_actuator[lane];
    double lo = m.actuator_ctrlrange[2 * act], hi = m.actuator_ctrlrange[2 * act + 1];
    double cl = isnan(t) ? t : fmin(hi, fmax(lo, t));
    ctrl[act] = (float)cl;
  }
  if (lane == 0) {
    double a6 = action[6];
    double sgn = isnan(a6) ? a6 : (a6 > 0 ? 1.0 : (a6 < 0 ? -1.0 : 0.0));
    double* grip = c.D(c.L.grip);
    for (int i = 0; i < 2; ++i) {
      double v = clip1(grip[i] + (double)m.osc_gripper_speed * (i == 0 ? -1.0 : 1.0) * sgn);
      grip[i] = v;
      int act = m.osc_actuator[7 + i];
      double lo = m.actuator_ctrlrange[2 * act], hi = m.actuator_ctrlrange[2 * act + 1];
      ctrl[act] = (float)((hi + lo) * 0.5 + (hi - lo) * 0.5 * v);
    }
  }
  sync();
}

// ---------------------------------------------------------------- actuation, smooth acceleration
// Joint-transmission actuators and qfrc_smooth, then qacc_smooth = M^-1 qfrc_smooth: reference
// gpu/cuda/fp32/fused_actuation_solve.cu:29-210 and gpu/cuda/dynamics/mjwarp_actuation.cu.
__device__ void actuation(const Ctx& c) {
  const MxModel& m = c.m;
  const float* qpos = c.F(c.L.qpos);
  const float* qvel = c.F(c.L.qvel);
  const float* ctrl = c.F(c.L.ctrl);
  bool off = m.opt_disableflags & (1 << 10);
  for (int a = c.lane; a < m.nu; a += kLanes) {
    float force = 0.f;
    if (!off) {
      int j = m.actuator_trnid[a], qa = m.jnt_qposadr[j], da = m.jnt_dofadr[j];
      float gear = m.actuator_gear[a], cv = ctrl[a];
      if (m.actuator_ctrllimited[a]) cv = fminf(fmaxf(cv, m.actuator_ctrlrange[2 * a]), m.actuator_ctrlrange[2 * a + 1]);
      float length = gear * qpos[qa], velocity = gear * qvel[da];
      force = m.actuator_gainprm[a] * cv;
      if (m.actuator_biastype[a] == 1)
        force += m.actuator_biasprm[3 * a] + m.actuator_biasprm[3 * a + 1] * length + m.actuator_biasprm[3 * a + 2] * velocity;
      if (m.actuator_forcelimited[a])
        force = fminf(fmaxf(force, m.actuator_forcerange[2 * a]), m.actuator_forcerange[2 * a + 1]);
    }
    c.F(c.L.actforce)[a] = force;
  }
  sync();
  for (int i = c.lane; i < m.nv; i += kLanes) {
    float qa = 0.f;
    if (!off)
      for (int a = 0; a < m.nu; ++a) {
        int j = m.actuator_trnid[a];
        if (m.jnt_dofadr[j] == i) qa += m.actuator_gear[a] * c.F(c.L.actforce)[a];
      }
    c.F(c.L.act)[i] = qa;
    float s = c.F(c.L.passive)[i] - c.F(c.L.bias)[i] + c.F(c.L.applied)[i] + qa;
    c.F(c.L.smooth)[i] = s;
    c.F(c.L.qacc_smooth)[i] = s;
  }
  sync();
  solve(c, c.F(c.L.L), c.F(c.L.qacc_smooth));
}

// ---------------------------------------------------------------- integration
// Semi-implicit Euler with implicit joint damping: MuJoCo mj_Euler; reference
// gpu/cuda/fp32/fused_euler_step.cu:35-269 and fused_tail.cu:15-90 (advance).
__device__ void euler(const Ctx& c) {
  const MxModel& m = c.m;
  const float h = m.opt_timestep;
  float* qvel = c.F(c.L.qvel);
  float* qpos = c.F(c.L.qpos);
  float* acc = c.F(c.L.tmp);
  bool damped = false;
  if (!(m.opt_disableflags & (1 << 15)))
    for (int i = 0; i < m.nv; ++i) damped |= m.dof_damping[i] > 0.f;
  if (damped) {
    factor(c, c.F(c.L.M), c.F(c.L.L), m.dof_damping, h);
    for (int i = c.lane; i < m.nv; i += kLanes) acc[i] = c.F(c.L.smooth)[i] + c.F(c.L.qcon)[i];
    sync();
    solve(c, c.F(c.L.L), acc);
  } else {
    for (int i = c.lane; i < m.nv; i += kLanes) acc[i] = c.F(c.L.qacc)[i];
    sync();
  }
  for (int i = c.lane; i < m.nv; i += kLanes) {
    c.F(c.L.warm)[i] = c.F(c.L.qacc)[i];
    qvel[i] += h * acc[i];
  }
  sync();
  for (int j = c.lane; j < m.njnt; j += kLanes) {
    int qa = m.jnt_qposadr[j], da = m.jnt_dofadr[j], type = m.jnt_type[j];
    if (type == 0) {
      for (int k = 0; k < 3; ++k) qpos[qa + k] += h * qvel[da + k];
      float* quat = qpos + qa + 3;
      float v[3] = {qvel[da + 3], qvel[da + 4], qvel[da + 5]};
      float nrm = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
      float axis[3] = {1.f, 0.f, 0.f}, angle = 0.f;
      if (nrm >= 1e-15f) { for (int k = 0; k < 3; ++k) axis[k] = v[k] / nrm; angle = h * nrm; }
      float s, co;
      sincosf(0.5f * angle, &s, &co);
      float qr[4] = {co, axis[0] * s, axis[1] * s, axis[2] * s};
      float qn[4] = {quat[0], quat[1], quat[2], quat[3]}, out[4];
      normalize4(qn);
      qmul(qn, qr, out);
      for (int k = 0; k < 4; ++k) quat[k] = out[k];
    } else if (type == 2 || type == 3) {
      qpos[qa] += h * qvel[da];
    }
  }
  sync();
}

// ---------------------------------------------------------------- kernel
__device__ void load_world(const Ctx& c) {
  const MxModel& m = c.m;
  const MxData& d = c.d;
  size_t w = c.w;
  for (int i = c.lane; i < m.nq; i += kLanes) c.F(c.L.qpos)[i] = d.qpos[w * m.nq + i];
  for (int i = c.lane; i < m.nv; i += kLanes) {
    c.F(c.L.qvel)[i] = d.qvel[w * m.nv + i];
    c.F(c.L.warm)[i] = d.qacc_warmstart[w * m.nv + i];
    c.F(c.L.applied)[i] = d.qfrc_applied[w * m.nv + i];
  }
  for (int i = c.lane; i < m.nu; i += kLanes) c.F(c.L.ctrl)[i] = d.ctrl[w * m.nu + i];
  if (c.lane < 3) c.D(c.L.goalpos)[c.lane] = d.osc_goal_pos[3 * w + c.lane];
  if (c.lane < 9) c.D(c.L.goalrot)[c.lane] = d.osc_goal_rot[9 * w + c.lane];
  if (c.lane < 2) c.D(c.L.grip)[c.lane] = d.osc_gripper[2 * w + c.lane];
  int* misc = reinterpret_cast<int*>(c.F(c.L.misc));
  if (c.lane < 16) misc[c.lane] = 0;
  sync();
  if (c.lane == 0) misc[kCtrlErr] = d.osc_error[w];
  sync();
}

template <typename Tv>
__device__ __forceinline__ void put(const Ctx& c, Tv* dst, const float* src, int width) {
  size_t base = (size_t)c.w * width;
  for (int i = c.lane; i < width; i += kLanes) dst[base + i] = src[i];
}

__device__ void publish_derived(const Ctx& c) {
  const MxModel& m = c.m;
  const MxData& d = c.d;
  int nv = m.nv, nb = m.nbody;
  put(c, d.qacc, c.F(c.L.qacc), nv);
  put(c, d.qacc_smooth, c.F(c.L.qacc_smooth), nv);
  put(c, d.qfrc_bias, c.F(c.L.bias), nv);
  put(c, d.qfrc_passive, c.F(c.L.passive), nv);
  put(c, d.qfrc_actuator, c.F(c.L.act), nv);
  put(c, d.qfrc_smooth, c.F(c.L.smooth), nv);
  put(c, d.qfrc_constraint, c.F(c.L.qcon), nv);
  put(c, d.actuator_force, c.F(c.L.actforce), m.nu);
  put(c, d.M, c.F(c.L.M), m.nM);
  put(c, d.xpos, c.F(c.L.xpos), 3 * nb);
  put(c, d.xquat, c.F(c.L.xquat), 4 * nb);
  put(c, d.xmat, c.F(c.L.xmat), 9 * nb);
  put(c, d.geom_xpos, c.F(c.L.gxpos), 3 * m.ngeom);
  put(c, d.geom_xmat, c.F(c.L.gxmat), 9 * m.ngeom);
  put(c, d.site_xpos, c.F(c.L.sxpos), 3 * m.nsite);
  put(c, d.site_xmat, c.F(c.L.sxmat), 9 * m.nsite);
  put(c, d.subtree_com, c.F(c.L.scom), 3 * nb);
}

__device__ void store_world(const Ctx& c, int integrated) {
  const MxModel& m = c.m;
  const MxData& d = c.d;
  size_t w = c.w;
  put(c, d.qpos, c.F(c.L.qpos), m.nq);
  put(c, d.qvel, c.F(c.L.qvel), m.nv);
  put(c, d.qacc_warmstart, c.F(c.L.warm), m.nv);
  put(c, d.ctrl, c.F(c.L.ctrl), m.nu);
  int* misc = reinterpret_cast<int*>(c.F(c.L.misc));
  if (c.lane < 3) d.osc_goal_pos[3 * w + c.lane] = c.D(c.L.goalpos)[c.lane];
  if (c.lane < 9) d.osc_goal_rot[9 * w + c.lane] = c.D(c.L.goalrot)[c.lane];
  if (c.lane < 2) d.osc_gripper[2 * w + c.lane] = c.D(c.L.grip)[c.lane];
  if (c.lane < 7) d.osc_tau[7 * w + c.lane] = c.D(c.L.tau)[c.lane];
  if (c.lane < 3) d.osc_rank[3 * w + c.lane] = misc[kRank0 + c.lane];
  if (c.lane == 0) {
    d.osc_error[w] = misc[kCtrlErr];
    d.nstep[w] += integrated;
    d.time[w] += integrated * m.opt_timestep;
  }
}

__global__ __launch_bounds__(kLanes) void control_step_kernel(MxModel m, MxData d, Layout L, int substeps,
                                                               int flags, const int32_t* mask) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int w = blockIdx.x;
  if (w >= d.nworld) return;
  if (mask && !mask[w]) return;
  Ctx c{m, d, L, reinterpret_cast<float*>(lds), reinterpret_cast<double*>(lds + L.dbase), w, (int)threadIdx.x};
  load_world(c);
  int integrated = 0;
  for (int s = 0; s < substeps; ++s) {
    const bool last = s == substeps - 1;
    const int policy = (flags & MX_FLAG_POLICY_FIRST) && s == 0;
    kinematics(c);
    com_pos(c);
    crb_mass(c);
    factor(c, c.F(L.M), c.F(L.L), nullptr, 0.f);
    velocity(c);
    if ((flags & MX_FLAG_BOOTSTRAP) && s == 0) {
      const float* sp = c.F(L.sxpos) + 3 * m.osc_site;
      const float* sr = c.F(L.sxmat) + 9 * m.osc_site;
      if (c.lane < 3) c.D(L.goalpos)[c.lane] = sp[c.lane];
      if (c.lane < 9) c.D(L.goalrot)[c.lane] = sr[c.lane];
      if (c.lane < 2) c.D(L.grip)[c.lane] = 0.0;
      if (c.lane == 0) reinterpret_cast<int*>(c.F(L.misc))[kCtrlErr] = 0;
      sync();
    }
    if (!(flags & MX_FLAG_NO_CONTROL)) control(c, policy, last);
    actuation(c);
    // constraint solve: models admitted by this build carry no constraint rows (njmax == 0)
    for (int i = c.lane; i < m.nv; i += kLanes) {
      c.F(L.qacc)[i] = c.F(L.qacc_smooth)[i];
      c.F(L.qcon)[i] = 0.f;
    }
    sync();
    if (last) publish_derived(c);
    if (flags & MX_FLAG_NO_INTEGRATE) break;
    euler(c);
    ++integrated;
  }
  store_world(c, integrated);
}

const char* kFieldTables[7][64] = {
#define N(name) #name,
    {MX_MODEL_REAL_ARRAYS(N)}, {MX_MODEL_INT_ARRAYS(N)}, {MX_MODEL_INT_SCALARS(N)},
    {MX_MODEL_REAL_SCALARS(N)}, {MX_DATA_REAL_ARRAYS(N)}, {MX_DATA_F64_ARRAYS(N)}, {MX_DATA_INT_ARRAYS(N)}
#undef N
};

int count_names(int which) {
  int n = 0;
  while (n < 64 && kFieldTables[which][n]) ++n;
  return n;
}

int device_lds_limit() {
  int dev = 0, value = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 65536;
  if (hipDeviceGetAttribute(&value, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) return 65536;
  return value;
}

int launch(const MxModel* m, const MxData* d, const int32_t* mask, int substeps, int flags, void* stream) {
  int rc = mx_check(m, d);
  if (rc) return rc;
  if (substeps < 1) return MX_ERR_INVALID;
  Layout L = make_layout(*m);
  if (L.bytes > device_lds_limit()) return MX_ERR_LDS;
  hipLaunchKernelGGL(control_step_kernel, dim3(d->nworld), dim3(kLanes), L.bytes, (hipStream_t)stream,
                     *m, *d, L, substeps, flags, mask);
  return (int)hipGetLastError();
}

}  // namespace mx

extern "C" {

int mx_abi_version(void) { return MX_ABI_VERSION; }
size_t mx_model_bytes(void) { return sizeof(MxModel); }
size_t mx_data_bytes(void) { return sizeof(MxData); }
int mx_arch(void) { return 950; }
const char* mx_source_id(void) { return "mx_step.hip:world-local-v3"; }

int mx_field_count(int which) { return which < 0 || which > 6 ? -1 : mx::count_names(which); }
const char* mx_field_name(int which, int index) {
  if (which < 0 || which > 6 || index < 0 || index >= mx::count_names(which)) return nullptr;
  return mx::kFieldTables[which][index];
}

int mx_check(const MxModel* m, const MxData* d) {
  if (!m || !d) return MX_ERR_INVALID;
  if (m->abi_version != MX_ABI_VERSION) return MX_ERR_INVALID;
  if (d->nworld < 1 || m->nq < 1 || m->nv < 1 || m->nbody < 2 || m->nu < 9 || m->nsite < 1 || m->ntree < 1)
    return MX_ERR_INVALID;
  if (m->nlevel < 1 || m->nM < 1 || m->nMpair < m->nv) return MX_ERR_INVALID;
  if (m->osc_site < 0 || m->osc_site >= m->nsite) return MX_ERR_INVALID;
  // this build admits constraint-free models only (constraints and contacts disabled)
  if (m->njmax != 0 || !(m->opt_disableflags & 1)) return MX_ERR_DOMAIN;
  const void* need[] = {d->time, d->qpos, d->qvel, d->ctrl, d->qacc_warmstart, d->qfrc_applied, d->qacc,
                        d->qacc_smooth, d->qfrc_bias, d->qfrc_passive, d->qfrc_actuator, d->qfrc_smooth,
                        d->qfrc_constraint, d->actuator_force, d->M, d->xpos, d->xquat, d->xmat,
                        d->geom_xpos, d->geom_xmat, d->site_xpos, d->site_xmat, d->subtree_com,
                        d->osc_mass, d->osc_jac, d->osc_q, d->osc_qvel, d->osc_bias, d->osc_ee_pos,
                        d->osc_ee_rot, d->osc_ee_vel, d->osc_action, d->osc_goal_pos, d->osc_goal_rot,
                        d->osc_gripper, d->osc_gains, d->osc_q0, d->osc_tau, d->overflow, d->osc_error,
                        d->osc_rank, d->nstep};
  for (const void* p : need)
    if (!p) return MX_ERR_INVALID;
  const void* mneed[] = {m->body_pos, m->body_quat, m->body_parent, m->level_adr, m->level_body, m->jnt_type,
                         m->dof_parent, m->tree_dofadr, m->mpair_i, m->mpair_j, m->osc_dofadr, m->osc_actuator};
  for (const void* p : mneed)
    if (!p) return MX_ERR_INVALID;
  return 0;
}

int mx_lds_bytes(const MxModel* m) { return m ? mx::make_layout(*m).bytes : MX_ERR_INVALID; }

int mx_control_step(const MxModel* m, const MxData* d, int substeps, int flags, void* stream) {
  return mx::launch(m, d, nullptr, substeps, flags & ~MX_FLAG_NO_INTEGRATE, stream);
}

int mx_forward(const MxModel* m, const MxData* d, const int32_t* mask, int flags, void* stream) {
  return mx::launch(m, d, mask, 1, (flags | MX_FLAG_NO_INTEGRATE) & ~MX_FLAG_POLICY_FIRST, stream);
}

const char* mx_error_string(int code) {
  switch (code) {
    case 0: return "success";
    case MX_ERR_INVALID: return "invalid argument";
    case MX_ERR_DOMAIN: return "model outside the admitted domain";
    case MX_ERR_LDS: return "per-world working set exceeds the LDS budget";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}
}
