// CPU FP64 oracle of the per-world control step -- TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// Serial, world-at-a-time C++ in double precision.  Each stage cites the reference file:line whose
// algorithm it restates.  The reference's own stages are MJWarp/MuJoCo algorithms; where the
// reference defers to MuJoCo (model compiler, spatial algebra), MuJoCo's published semantics are
// restated (mj_kinematics, mj_comPos, mj_crb, mj_comVel, mj_rne, mj_passive, mj_fwdActuation,
// mj_Euler).  Nothing here is shipped or called by the product path.
#include "oracle_internal.h"

#include <atomic>
#include <thread>
#include <sched.h>

namespace orc {

// spatial algebra in MuJoCo's [angular; linear] convention
inline void mul_inert_vec(const T* i, const T* v, T* r) {
  r[0] = i[0] * v[0] + i[3] * v[1] + i[4] * v[2] - i[8] * v[4] + i[7] * v[5];
  r[1] = i[3] * v[0] + i[1] * v[1] + i[5] * v[2] + i[8] * v[3] - i[6] * v[5];
  r[2] = i[4] * v[0] + i[5] * v[1] + i[2] * v[2] - i[7] * v[3] + i[6] * v[4];
  r[3] = i[8] * v[1] - i[7] * v[2] + i[9] * v[3];
  r[4] = i[6] * v[2] - i[8] * v[0] + i[9] * v[4];
  r[5] = i[7] * v[0] - i[6] * v[1] + i[9] * v[5];
}
inline void cross_motion(const T* v, const T* u, T* r) {
  r[0] = -v[2] * u[1] + v[1] * u[2];
  r[1] = v[2] * u[0] - v[0] * u[2];
  r[2] = -v[1] * u[0] + v[0] * u[1];
  r[3] = -v[2] * u[4] + v[1] * u[5] - v[5] * u[1] + v[4] * u[2];
  r[4] = v[2] * u[3] - v[0] * u[5] + v[5] * u[0] - v[3] * u[2];
  r[5] = -v[1] * u[3] + v[0] * u[4] - v[4] * u[0] + v[3] * u[1];
}
inline void cross_force(const T* v, const T* f, T* r) {
  r[0] = -v[2] * f[1] + v[1] * f[2] - v[5] * f[4] + v[4] * f[5];
  r[1] = v[2] * f[0] - v[0] * f[2] + v[5] * f[3] - v[3] * f[5];
  r[2] = -v[1] * f[0] + v[0] * f[1] - v[4] * f[3] + v[3] * f[4];
  r[3] = -v[2] * f[4] + v[1] * f[5];
  r[4] = v[2] * f[3] - v[0] * f[5];
  r[5] = -v[1] * f[3] + v[0] * f[4];
}

World::World(const OrModel& m) {
  int nb = m.nbody, nv = m.nv, nj = m.njnt;
  xpos.assign(3 * nb, 0); xquat.assign(4 * nb, 0); xmat.assign(9 * nb, 0);
  xipos.assign(3 * nb, 0); ximat.assign(9 * nb, 0); xanchor.assign(3 * nj, 0); xaxis.assign(3 * nj, 0);
  subtree_com.assign(3 * nb, 0); cinert.assign(10 * nb, 0); crb.assign(10 * nb, 0);
  cdof.assign(6 * nv, 0); cvel.assign(6 * nb, 0); cdof_dot.assign(6 * nv, 0);
  cacc.assign(6 * nb, 0); cfrc.assign(6 * nb, 0); M.assign(m.nM, 0); L.assign(m.nM, 0); L2.assign(m.nM, 0);
  geom_xpos.assign(3 * m.ngeom, 0); geom_xmat.assign(9 * m.ngeom, 0);
  site_xpos.assign(3 * m.nsite, 0); site_xmat.assign(9 * m.nsite, 0);
  qfrc_bias.assign(nv, 0); qfrc_passive.assign(nv, 0); qfrc_actuator.assign(nv, 0);
  qfrc_smooth.assign(nv, 0); qacc_smooth.assign(nv, 0); qacc.assign(nv, 0); qfrc_constraint.assign(nv, 0);
  actuator_force.assign(m.nu, 0); jacp.assign(3 * nv, 0); jacr.assign(3 * nv, 0); tmp.assign(nv, 0);
  qfrc_gravcomp.assign(nv, 0); qfrc_xfrc.assign(nv, 0);
  cfrc_ext.assign(6 * nb, 0); cacc_post.assign(6 * nb, 0); cfrc_int.assign(6 * nb, 0);
  Ma.assign(nv, 0); grad.assign(nv, 0); search.assign(nv, 0); Mv.assign(nv, 0);
  H.assign((size_t)nv * nv, 0); Hf.assign((size_t)nv * nv, 0);
}

// ------------------------------------------------------------------ position stage
// Forward kinematics: MuJoCo mj_kinematics semantics; reference fused leaf
// gpu/cuda/fp32/fused_kinematic_mass.cu:110-447 (joint deltas, body/inertial/geom/site frames).
void kinematics(const OrModel& m, const T* qpos, World& w) {
  w.xpos[0] = w.xpos[1] = w.xpos[2] = 0;
  w.xquat[0] = 1; w.xquat[1] = w.xquat[2] = w.xquat[3] = 0;
  for (int k = 0; k < 9; ++k) w.xmat[k] = (k % 4 == 0) ? 1 : 0;
  for (int b = 1; b < m.nbody; ++b) {
    int p = m.body_parent[b];
    T pos[3], quat[4], off[3];
    mulmv3(&w.xmat[9 * p], m.body_pos + 3 * b, off);
    for (int k = 0; k < 3; ++k) pos[k] = w.xpos[3 * p + k] + off[k];
    qmul(&w.xquat[4 * p], m.body_quat + 4 * b, quat);
    for (int j = m.body_jntadr[b]; j < m.body_jntadr[b] + m.body_jntnum[b]; ++j) {
      int qa = m.jnt_qposadr[j], type = m.jnt_type[j];
      if (type == 0) {  // free
        for (int k = 0; k < 3; ++k) pos[k] = qpos[qa + k];
        for (int k = 0; k < 4; ++k) quat[k] = qpos[qa + 3 + k];
        normalize4(quat);
        for (int k = 0; k < 3; ++k) w.xanchor[3 * j + k] = pos[k];
        w.xaxis[3 * j] = 0; w.xaxis[3 * j + 1] = 0; w.xaxis[3 * j + 2] = 1;
        continue;
      }
      T R[9], anc[3], ax[3];
      quat2mat(quat, R);
      mulmv3(R, m.jnt_pos + 3 * j, anc);
      for (int k = 0; k < 3; ++k) anc[k] += pos[k];
      mulmv3(R, m.jnt_axis + 3 * j, ax);
      for (int k = 0; k < 3; ++k) { w.xanchor[3 * j + k] = anc[k]; w.xaxis[3 * j + k] = ax[k]; }
      T delta = qpos[qa] - m.qpos0[qa];
      if (type == 2) {  // slide
        for (int k = 0; k < 3; ++k) pos[k] += ax[k] * delta;
      } else if (type == 3) {  // hinge: rotate about the anchor
        T s = std::sin(delta / 2), ql[4] = {std::cos(delta / 2), m.jnt_axis[3 * j] * s,
                                            m.jnt_axis[3 * j + 1] * s, m.jnt_axis[3 * j + 2] * s};
        T nq[4];
        qmul(quat, ql, nq);
        std::memcpy(quat, nq, sizeof nq);
        quat2mat(quat, R);
        T r[3];
        mulmv3(R, m.jnt_pos + 3 * j, r);
        for (int k = 0; k < 3; ++k) pos[k] = anc[k] - r[k];
      }
    }
    normalize4(quat);
    for (int k = 0; k < 3; ++k) w.xpos[3 * b + k] = pos[k];
    for (int k = 0; k < 4; ++k) w.xquat[4 * b + k] = quat[k];
    quat2mat(quat, &w.xmat[9 * b]);
  }
  for (int b = 0; b < m.nbody; ++b) {
    T off[3], R[9];
    mulmv3(&w.xmat[9 * b], m.body_ipos + 3 * b, off);
    for (int k = 0; k < 3; ++k) w.xipos[3 * b + k] = w.xpos[3 * b + k] + off[k];
    quat2mat(m.body_iquat + 4 * b, R);
    mulmm3(&w.xmat[9 * b], R, &w.ximat[9 * b]);
  }
  for (int g = 0; g < m.ngeom; ++g) {
    int b = m.geom_body[g];
    T off[3], R[9];
    mulmv3(&w.xmat[9 * b], m.geom_pos + 3 * g, off);
    for (int k = 0; k < 3; ++k) w.geom_xpos[3 * g + k] = w.xpos[3 * b + k] + off[k];
    quat2mat(m.geom_quat + 4 * g, R);
    mulmm3(&w.xmat[9 * b], R, &w.geom_xmat[9 * g]);
  }
  for (int s = 0; s < m.nsite; ++s) {
    int b = m.site_body[s];
    T off[3], R[9];
    mulmv3(&w.xmat[9 * b], m.site_pos + 3 * s, off);
    for (int k = 0; k < 3; ++k) w.site_xpos[3 * s + k] = w.xpos[3 * b + k] + off[k];
    quat2mat(m.site_quat + 4 * s, R);
    mulmm3(&w.xmat[9 * b], R, &w.site_xmat[9 * s]);
  }
}

// Subtree centres of mass, cinert and cdof: MuJoCo mj_comPos; reference
// gpu/cuda/dynamics/mjwarp_com_pos.cu:95 (centered_frames) and fused_kinematic_mass.cu.
void com_pos(const OrModel& m, World& w) {
  int nb = m.nbody;
  for (int b = 0; b < nb; ++b)
    for (int k = 0; k < 3; ++k) w.subtree_com[3 * b + k] = w.xipos[3 * b + k] * m.body_mass[b];
  for (int b = nb - 1; b > 0; --b)
    for (int k = 0; k < 3; ++k) w.subtree_com[3 * m.body_parent[b] + k] += w.subtree_com[3 * b + k];
  for (int b = 0; b < nb; ++b) {
    if (m.body_subtreemass[b] < kMinVal)
      for (int k = 0; k < 3; ++k) w.subtree_com[3 * b + k] = w.xipos[3 * b + k];
    else
      for (int k = 0; k < 3; ++k) w.subtree_com[3 * b + k] /= m.body_subtreemass[b];
  }
  for (int k = 0; k < 10; ++k) w.cinert[k] = 0;
  for (int b = 1; b < nb; ++b) {
    const T* R = &w.ximat[9 * b];
    const T* I = m.body_inertia + 3 * b;
    T mass = m.body_mass[b], d[3];
    int r = m.body_rootid[b];
    for (int k = 0; k < 3; ++k) d[k] = w.xipos[3 * b + k] - w.subtree_com[3 * r + k];
    T* c = &w.cinert[10 * b];
    // rotational inertia R diag(I) R^T about the body com, then the parallel-axis shift
    T rot[9];
    for (int i = 0; i < 3; ++i)
      for (int j = 0; j < 3; ++j)
        rot[3 * i + j] = R[3 * i] * I[0] * R[3 * j] + R[3 * i + 1] * I[1] * R[3 * j + 1] + R[3 * i + 2] * I[2] * R[3 * j + 2];
    c[0] = rot[0] + mass * (d[1] * d[1] + d[2] * d[2]);
    c[1] = rot[4] + mass * (d[0] * d[0] + d[2] * d[2]);
    c[2] = rot[8] + mass * (d[0] * d[0] + d[1] * d[1]);
    c[3] = rot[1] - mass * d[0] * d[1];
    c[4] = rot[2] - mass * d[0] * d[2];
    c[5] = rot[5] - mass * d[1] * d[2];
    c[6] = mass * d[0]; c[7] = mass * d[1]; c[8] = mass * d[2]; c[9] = mass;
  }
  for (int j = 0; j < m.njnt; ++j) {
    int b = m.jnt_body[j], da = m.jnt_dofadr[j], r = m.body_rootid[b];
    T off[3];
    for (int k = 0; k < 3; ++k) off[k] = w.subtree_com[3 * r + k] - w.xanchor[3 * j + k];
    const T* ax = &w.xaxis[3 * j];
    switch (m.jnt_type[j]) {
      case 0:  // free: 3 world translations, then rotations about the body's own axes
        for (int d = 0; d < 3; ++d) {
          T* c = &w.cdof[6 * (da + d)];
          for (int k = 0; k < 6; ++k) c[k] = 0;
          c[3 + d] = 1;
        }
        for (int d = 0; d < 3; ++d) {
          T* c = &w.cdof[6 * (da + 3 + d)];
          T a[3] = {w.xmat[9 * b + d], w.xmat[9 * b + 3 + d], w.xmat[9 * b + 6 + d]};
          c[0] = a[0]; c[1] = a[1]; c[2] = a[2];
          cross(a, off, c + 3);
        }
        break;
      case 2: {  // slide
        T* c = &w.cdof[6 * da];
        c[0] = c[1] = c[2] = 0; c[3] = ax[0]; c[4] = ax[1]; c[5] = ax[2];
        break;
      }
      case 3: {  // hinge
        T* c = &w.cdof[6 * da];
        c[0] = ax[0]; c[1] = ax[1]; c[2] = ax[2];
        cross(ax, off, c + 3);
        break;
      }
      default: break;
    }
  }
}

// Composite rigid body mass matrix in dense per-tree blocks: MuJoCo mj_crb; reference
// fused_kinematic_mass.cu (CRB, M rows) and gpu/cuda/dynamics/mjwarp_mass_matrix.cu:54.
void crb(const OrModel& m, World& w) {
  std::copy(w.cinert.begin(), w.cinert.end(), w.crb.begin());
  for (int b = m.nbody - 1; b > 0; --b)
    if (m.body_parent[b] > 0)
      for (int k = 0; k < 10; ++k) w.crb[10 * m.body_parent[b] + k] += w.crb[10 * b + k];
  std::fill(w.M.begin(), w.M.end(), 0.0);
  for (int i = 0; i < m.nv; ++i) {
    T buf[6];
    mul_inert_vec(&w.crb[10 * m.dof_body[i]], &w.cdof[6 * i], buf);
    int t = m.dof_treeid[i], n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    T* blk = &w.M[m.tree_madr[t]];
    for (int j = i; j >= 0; j = m.dof_parent[j]) {
      T v = 0;
      for (int k = 0; k < 6; ++k) v += w.cdof[6 * j + k] * buf[k];
      if (j == i) v += m.dof_armature[i];
      blk[(i - a) * n + (j - a)] = v;
      blk[(j - a) * n + (i - a)] = v;
    }
  }
}

// Per-tree dense Cholesky M = L L^T (lower, row-major in the block storage); reference
// gpu/cuda/dynamics/mjwarp_mass_factor.cu:134-247 (per-tree block factorization).
// diag_add (may be null) is added to the diagonal first (implicit damping, fused_euler_step.cu).
void factor(const OrModel& m, const T* M, T* L, const T* diag_add, T scale) {
  for (int t = 0; t < m.ntree; ++t) {
    int n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    const T* A = M + m.tree_madr[t];
    T* F = L + m.tree_madr[t];
    for (int k = 0; k < n * n; ++k) F[k] = A[k];
    if (diag_add)
      for (int i = 0; i < n; ++i) F[i * n + i] += scale * diag_add[a + i];
    for (int j = 0; j < n; ++j) {
      T d = F[j * n + j];
      for (int k = 0; k < j; ++k) d -= F[j * n + k] * F[j * n + k];
      d = std::sqrt(std::max(d, kMinVal));
      F[j * n + j] = d;
      for (int i = j + 1; i < n; ++i) {
        T v = F[i * n + j];
        for (int k = 0; k < j; ++k) v -= F[i * n + k] * F[j * n + k];
        F[i * n + j] = v / d;
      }
    }
  }
}

// x <- M^-1 x with the per-tree factor (POTRS role of gpu/cuda/dynamics/mjwarp_mass_solve.cu:74-122).
void solve(const OrModel& m, const T* L, T* x) {
  for (int t = 0; t < m.ntree; ++t) {
    int n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    const T* F = L + m.tree_madr[t];
    T* v = x + a;
    for (int i = 0; i < n; ++i) {
      T s = v[i];
      for (int k = 0; k < i; ++k) s -= F[i * n + k] * v[k];
      v[i] = s / F[i * n + i];
    }
    for (int i = n - 1; i >= 0; --i) {
      T s = v[i];
      for (int k = i + 1; k < n; ++k) s -= F[k * n + i] * v[k];
      v[i] = s / F[i * n + i];
    }
  }
}

// ------------------------------------------------------------------ velocity stage
// cvel and cdof_dot: MuJoCo mj_comVel; reference gpu/cuda/dynamics/mjwarp_velocity.cu and
// gpu/cuda/fp32/fused_motion_passive.cu:43-387 (cvel, cdof_dot).
void com_vel(const OrModel& m, const T* qvel, World& w) {
  for (int k = 0; k < 6; ++k) w.cvel[k] = 0;
  for (int b = 1; b < m.nbody; ++b) {
    T v[6];
    for (int k = 0; k < 6; ++k) v[k] = w.cvel[6 * m.body_parent[b] + k];
    for (int j = m.body_jntadr[b]; j < m.body_jntadr[b] + m.body_jntnum[b]; ++j) {
      int da = m.jnt_dofadr[j];
      int ndof = m.jnt_type[j] == 0 ? 6 : (m.jnt_type[j] == 1 ? 3 : 1);
      int first = 0;
      if (m.jnt_type[j] == 0) {  // translations: cdof_dot = 0
        for (int d = 0; d < 3; ++d) {
          for (int k = 0; k < 6; ++k) w.cdof_dot[6 * (da + d) + k] = 0;
          for (int k = 0; k < 6; ++k) v[k] += w.cdof[6 * (da + d) + k] * qvel[da + d];
        }
        first = 3;
      }
      if (ndof - first == 3) {  // rotations of a free (or ball) joint: use the same velocity
        for (int d = first; d < ndof; ++d) cross_motion(v, &w.cdof[6 * (da + d)], &w.cdof_dot[6 * (da + d)]);
        for (int d = first; d < ndof; ++d)
          for (int k = 0; k < 6; ++k) v[k] += w.cdof[6 * (da + d) + k] * qvel[da + d];
      } else if (ndof == 1) {
        cross_motion(v, &w.cdof[6 * da], &w.cdof_dot[6 * da]);
        for (int k = 0; k < 6; ++k) v[k] += w.cdof[6 * da + k] * qvel[da];
      }
    }
    for (int k = 0; k < 6; ++k) w.cvel[6 * b + k] = v[k];
  }
}

// Recursive Newton-Euler bias forces (no acceleration): MuJoCo mj_rne(flg_acc=0); reference
// gpu/cuda/fp32/fused_motion.cu:14 (motion_bias) and gpu/cuda/dynamics/mjwarp_bias.cu.
void rne(const OrModel& m, const T* qvel, World& w) {
  T* cacc = w.cacc.data();
  for (int k = 0; k < 6; ++k) cacc[k] = 0;
  if (!(m.opt_disableflags & (1 << 6))) {
    cacc[3] = -m.opt_gravity_x; cacc[4] = -m.opt_gravity_y; cacc[5] = -m.opt_gravity_z;
  }
  for (int k = 0; k < 6; ++k) w.cfrc[k] = 0;
  for (int b = 1; b < m.nbody; ++b) {
    int p = m.body_parent[b];
    for (int k = 0; k < 6; ++k) cacc[6 * b + k] = cacc[6 * p + k];
    for (int d = m.body_dofadr[b]; d < m.body_dofadr[b] + m.body_dofnum[b]; ++d)
      for (int k = 0; k < 6; ++k) cacc[6 * b + k] += w.cdof_dot[6 * d + k] * qvel[d];
    T f1[6], h[6], f2[6];
    mul_inert_vec(&w.cinert[10 * b], &cacc[6 * b], f1);
    mul_inert_vec(&w.cinert[10 * b], &w.cvel[6 * b], h);
    cross_force(&w.cvel[6 * b], h, f2);
    for (int k = 0; k < 6; ++k) w.cfrc[6 * b + k] = f1[k] + f2[k];
  }
  for (int b = m.nbody - 1; b > 0; --b)
    if (m.body_parent[b] > 0)
      for (int k = 0; k < 6; ++k) w.cfrc[6 * m.body_parent[b] + k] += w.cfrc[6 * b + k];
  for (int i = 0; i < m.nv; ++i) {
    T s = 0;
    for (int k = 0; k < 6; ++k) s += w.cdof[6 * i + k] * w.cfrc[6 * m.dof_body[i] + k];
    w.qfrc_bias[i] = s;
  }
}

// Joint springs and dampers: MuJoCo mj_passive; reference gpu/cuda/dynamics/mjwarp_passive.cu:15,52.
void passive(const OrModel& m, const T* qpos, const T* qvel, World& w) {
  std::fill(w.qfrc_passive.begin(), w.qfrc_passive.end(), 0.0);
  if (m.opt_disableflags & (1 << 5)) return;
  for (int j = 0; j < m.njnt; ++j) {
    int type = m.jnt_type[j];
    if ((type == 2 || type == 3) && m.jnt_stiffness[j] != 0) {
      int qa = m.jnt_qposadr[j];
      w.qfrc_passive[m.jnt_dofadr[j]] -= m.jnt_stiffness[j] * (qpos[qa] - m.qpos_spring[qa]);
    }
  }
  for (int i = 0; i < m.nv; ++i) w.qfrc_passive[i] -= m.dof_damping[i] * qvel[i];
}

// Gravity compensation: generalized force of -gravity * mass * gravcomp at each body's centre of
// mass (MuJoCo mj_gravcomp; reference gpu/cuda/dynamics/mjwarp_queries.cu:55 rigid_gravity_projection),
// added to the passive force of dofs whose joint does not report it as actuator force
// (mjwarp_passive.cu:57) and to the actuator force of the others (mjwarp_actuation.cu:54).
void gravcomp(const OrModel& m, World& w) {
  std::fill(w.qfrc_gravcomp.begin(), w.qfrc_gravcomp.end(), 0.0);
  if (!m.has_gravcomp || (m.opt_disableflags & (1 << 6))) return;
  const T g[3] = {m.opt_gravity_x, m.opt_gravity_y, m.opt_gravity_z};
  for (int b = 1; b < m.nbody; ++b) {
    T c = m.body_gravcomp[b];
    if (c == 0) continue;
    T f[3];
    for (int k = 0; k < 3; ++k) f[k] = -g[k] * m.body_mass[b] * c;
    body_jac(m, w, b, &w.xipos[3 * b], w.jacp.data(), w.jacr.data());
    for (int d = 0; d < m.nv; ++d)
      for (int k = 0; k < 3; ++k) w.qfrc_gravcomp[d] += w.jacp[k * m.nv + d] * f[k];
  }
  for (int d = 0; d < m.nv; ++d)
    if (!m.jnt_actgravcomp[m.dof_jnt[d]]) w.qfrc_passive[d] += w.qfrc_gravcomp[d];
}

// Fluid forces of MuJoCo's inertia-box model (mj_passive -> mj_inertiaBoxFluidModel; reference
// gpu/cuda/fp32/fused_motion_passive.cu:253-330 and the dof projection :350-372): each body with
// mass drags through the medium as the box of its principal inertia, side_k =
// sqrt(6 (I_i + I_j - I_k) / mass).  In the inertial frame, with v the centre-of-mass velocity
// relative to the wind and w the angular velocity: Stokes terms -3 pi mu d v and -pi mu d^3 w
// (d the mean side) and quadratic terms -rho/2 s_i s_j |v_k| v_k and
// -rho/64 s_k (s_i^4 + s_j^4) |w_k| w_k; the wrench at the centre of mass goes into the passive
// force.  The body velocity is taken here from the point Jacobian (the kernel uses cvel).
void fluid(const OrModel& m, const T* qvel, World& w) {
  if (!m.has_fluid || (m.opt_disableflags & (1 << 5))) return;
  const T pi = 3.14159265358979323846;
  for (int b = 1; b < m.nbody; ++b) {
    T mass = m.body_mass[b];
    if (mass < 1e-15) continue;
    body_jac(m, w, b, &w.xipos[3 * b], w.jacp.data(), w.jacr.data());
    T v[3] = {0, 0, 0}, om[3] = {0, 0, 0};
    for (int k = 0; k < 3; ++k)
      for (int d = 0; d < m.nv; ++d) {
        v[k] += w.jacp[k * m.nv + d] * qvel[d];
        om[k] += w.jacr[k * m.nv + d] * qvel[d];
      }
    v[0] -= m.opt_wind_x; v[1] -= m.opt_wind_y; v[2] -= m.opt_wind_z;
    const T* R = &w.ximat[9 * b];
    T lv[3], lw[3];
    for (int k = 0; k < 3; ++k) {
      lv[k] = R[k] * v[0] + R[3 + k] * v[1] + R[6 + k] * v[2];
      lw[k] = R[k] * om[0] + R[3 + k] * om[1] + R[6 + k] * om[2];
    }
    const T* I = m.body_inertia + 3 * b;
    T s[3];
    for (int k = 0; k < 3; ++k)
      s[k] = std::sqrt(std::max<T>(1e-15, I[(k + 1) % 3] + I[(k + 2) % 3] - I[k]) * 6.0 / mass);
    T lf[3] = {0, 0, 0}, lt[3] = {0, 0, 0};
    if (m.opt_viscosity > 0) {
      T d = (s[0] + s[1] + s[2]) / 3.0;
      for (int k = 0; k < 3; ++k) {
        lf[k] = -3.0 * pi * m.opt_viscosity * d * lv[k];
        lt[k] = -pi * m.opt_viscosity * d * d * d * lw[k];
      }
    }
    if (m.opt_density > 0) {
      for (int k = 0; k < 3; ++k) {
        T si = s[(k + 1) % 3], sj = s[(k + 2) % 3];
        lf[k] -= 0.5 * m.opt_density * si * sj * std::fabs(lv[k]) * lv[k];
        lt[k] -= m.opt_density / 64.0 * s[k] * (std::pow(si, 4) + std::pow(sj, 4)) * std::fabs(lw[k]) * lw[k];
      }
    }
    T f[3], t[3];
    for (int k = 0; k < 3; ++k) {
      f[k] = R[3 * k] * lf[0] + R[3 * k + 1] * lf[1] + R[3 * k + 2] * lf[2];
      t[k] = R[3 * k] * lt[0] + R[3 * k + 1] * lt[1] + R[3 * k + 2] * lt[2];
    }
    for (int d = 0; d < m.nv; ++d)
      for (int k = 0; k < 3; ++k) w.qfrc_passive[d] += w.jacp[k * m.nv + d] * f[k] + w.jacr[k * m.nv + d] * t[k];
  }
}

// Applied Cartesian wrenches xfrc_applied (force, torque at each body's centre of mass, world
// frame) projected on the dofs: MuJoCo mj_xfrcAccumulate, added to qfrc_smooth.
void xfrc_project(const OrModel& m, const T* xfrc, World& w) {
  std::fill(w.qfrc_xfrc.begin(), w.qfrc_xfrc.end(), 0.0);
  for (int b = 1; b < m.nbody; ++b) {
    const T* x = xfrc + 6 * b;
    if (!x[0] && !x[1] && !x[2] && !x[3] && !x[4] && !x[5]) continue;
    body_jac(m, w, b, &w.xipos[3 * b], w.jacp.data(), w.jacr.data());
    for (int d = 0; d < m.nv; ++d)
      for (int k = 0; k < 3; ++k) w.qfrc_xfrc[d] += w.jacp[k * m.nv + d] * x[k] + w.jacr[k * m.nv + d] * x[3 + k];
  }
}

// cfrc_ext, cacc, cfrc_int and force / torque sensors after the constraint solve (reference
// gpu/cuda/dynamics/mjwarp_external_wrench.cu:26-90 initialize_applied / accumulate_contacts,
// mjwarp_postconstraint.cu:87 world_postconstraint, mjwarp_queries.cu:31 force_torque_sensors).
// Spatial quantities are [torque; force] about the subtree centre of mass of the body's root.
void post_constraint(const OrModel& m, const T* qvel, const T* xfrc, World& w, T* sensordata) {
  int nb = m.nbody;
  std::fill(w.cfrc_ext.begin(), w.cfrc_ext.end(), 0.0);
  for (int b = 1; b < nb; ++b) {
    const T* x = xfrc + 6 * b;
    const T* c = &w.subtree_com[3 * m.body_rootid[b]];
    T off[3] = {w.xipos[3 * b] - c[0], w.xipos[3 * b + 1] - c[1], w.xipos[3 * b + 2] - c[2]}, t[3];
    cross(off, x, t);
    for (int k = 0; k < 3; ++k) { w.cfrc_ext[6 * b + k] = x[3 + k] + t[k]; w.cfrc_ext[6 * b + 3 + k] = x[k]; }
  }
  for (const Contact& ct : w.contacts) {
    if (ct.efc_address < 0) continue;
    T local[3] = {0, 0, 0};
    const T* f = &w.force[ct.efc_address];
    if (ct.dim == 1) local[0] = f[0];
    else if (m.opt_cone == 0) {          // pyramidal: edge pairs (n + mu t, n - mu t)
      for (int i = 0; i < ct.dim - 1; ++i) {
        local[0] += f[2 * i] + f[2 * i + 1];
        local[i + 1] = (f[2 * i] - f[2 * i + 1]) * ct.friction[i];
      }
    } else {
      for (int i = 0; i < ct.dim; ++i) local[i] = f[i];
    }
    T F[3];
    mulmtv3(ct.frame, local, F);         // frame rows: normal, tangent 1, tangent 2
    int bodies[2] = {m.geom_body[ct.geom[0]], m.geom_body[ct.geom[1]]};
    for (int side = 0; side < 2; ++side) {
      int b = bodies[side];
      if (b == 0) continue;
      const T* c = &w.subtree_com[3 * m.body_rootid[b]];
      T off[3] = {ct.pos[0] - c[0], ct.pos[1] - c[1], ct.pos[2] - c[2]}, t[3];
      cross(off, F, t);
      T sign = side == 0 ? -1 : 1;
      for (int k = 0; k < 3; ++k) { w.cfrc_ext[6 * b + k] += sign * t[k]; w.cfrc_ext[6 * b + 3 + k] += sign * F[k]; }
    }
  }
  T* cacc = w.cacc_post.data();
  for (int k = 0; k < 6; ++k) cacc[k] = 0;
  if (!(m.opt_disableflags & (1 << 6))) {
    cacc[3] = -m.opt_gravity_x; cacc[4] = -m.opt_gravity_y; cacc[5] = -m.opt_gravity_z;
  }
  for (int k = 0; k < 6; ++k) w.cfrc_int[k] = 0;
  for (int b = 1; b < nb; ++b) {
    int p = m.body_parent[b];
    for (int k = 0; k < 6; ++k) cacc[6 * b + k] = cacc[6 * p + k];
    for (int d = m.body_dofadr[b]; d < m.body_dofadr[b] + m.body_dofnum[b]; ++d)
      for (int k = 0; k < 6; ++k) cacc[6 * b + k] += w.cdof_dot[6 * d + k] * qvel[d] + w.cdof[6 * d + k] * w.qacc[d];
    T f1[6], h[6], f2[6];
    mul_inert_vec(&w.cinert[10 * b], &cacc[6 * b], f1);
    mul_inert_vec(&w.cinert[10 * b], &w.cvel[6 * b], h);
    cross_force(&w.cvel[6 * b], h, f2);
    for (int k = 0; k < 6; ++k) w.cfrc_int[6 * b + k] = f1[k] + f2[k] - w.cfrc_ext[6 * b + k];
  }
  for (int b = nb - 1; b > 0; --b)
    if (m.body_parent[b] > 0)
      for (int k = 0; k < 6; ++k) w.cfrc_int[6 * m.body_parent[b] + k] += w.cfrc_int[6 * b + k];
  for (int s = 0; s < m.nsensor; ++s) {
    int site = m.sensor_objid[s], b = m.site_body[site];
    const T* wr = &w.cfrc_int[6 * b];
    T value[3];
    if (m.sensor_type[s] == MX_SENS_FORCE) {
      for (int k = 0; k < 3; ++k) value[k] = wr[3 + k];
    } else {
      const T* c = &w.subtree_com[3 * m.body_rootid[b]];
      T off[3] = {w.site_xpos[3 * site] - c[0], w.site_xpos[3 * site + 1] - c[1], w.site_xpos[3 * site + 2] - c[2]}, t[3];
      cross(off, wr + 3, t);
      for (int k = 0; k < 3; ++k) value[k] = wr[k] - t[k];
    }
    T out[3];
    mulmtv3(&w.site_xmat[9 * site], value, out);
    T cut = m.sensor_cutoff[s];
    for (int k = 0; k < 3; ++k) {
      if (cut > 0) {
        if (m.sensor_datatype[s] == 0) out[k] = std::min(cut, std::max(-cut, out[k]));
        else if (m.sensor_datatype[s] == 1) out[k] = std::min(cut, out[k]);
      }
      sensordata[m.sensor_adr[s] + k] = out[k];
    }
  }
}

// Site Jacobian (translational, rotational): MuJoCo mj_jac; reference
// gpu/cuda/dynamics/mjwarp_queries.cu:19 (point_jacobians) and fused_control_drive.cu.
void site_jac(const OrModel& m, const World& w, int site, T* jacp, T* jacr) {
  int b = m.site_body[site], r = m.body_rootid[b];
  T off[3];
  for (int k = 0; k < 3; ++k) off[k] = w.site_xpos[3 * site + k] - w.subtree_com[3 * r + k];
  std::fill(jacp, jacp + 3 * m.nv, 0.0);
  std::fill(jacr, jacr + 3 * m.nv, 0.0);
  for (int d = m.body_lastdof[b]; d >= 0; d = m.dof_parent[d]) {
    const T* c = &w.cdof[6 * d];
    T t[3];
    cross(c, off, t);
    for (int k = 0; k < 3; ++k) {
      jacr[k * m.nv + d] = c[k];
      jacp[k * m.nv + d] = c[3 + k] + t[k];
    }
  }
}

// Actuation with joint transmission: MuJoCo mj_transmission + mj_fwdActuation; reference
// gpu/cuda/dynamics/mjwarp_transmission.cu:41 and gpu/cuda/fp32/fused_actuation_solve.cu:29-210.
void actuation(const OrModel& m, const T* qpos, const T* qvel, T* ctrl, World& w) {
  std::fill(w.qfrc_actuator.begin(), w.qfrc_actuator.end(), 0.0);
  if (m.opt_disableflags & (1 << 10)) {
    std::fill(w.actuator_force.begin(), w.actuator_force.end(), 0.0);
    return;
  }
  for (int a = 0; a < m.nu; ++a) {
    int j = m.actuator_trnid[a], qa = m.jnt_qposadr[j], da = m.jnt_dofadr[j];
    T gear = m.actuator_gear[a];
    T c = ctrl[a];
    if (m.actuator_ctrllimited[a]) c = std::min(std::max(c, m.actuator_ctrlrange[2 * a]), m.actuator_ctrlrange[2 * a + 1]);
    T length = gear * qpos[qa], velocity = gear * qvel[da];
    T force = m.actuator_gainprm[a] * c;
    if (m.actuator_biastype[a] == 1)
      force += m.actuator_biasprm[3 * a] + m.actuator_biasprm[3 * a + 1] * length + m.actuator_biasprm[3 * a + 2] * velocity;
    if (m.actuator_forcelimited[a])
      force = std::min(std::max(force, m.actuator_forcerange[2 * a]), m.actuator_forcerange[2 * a + 1]);
    w.actuator_force[a] = force;
    w.qfrc_actuator[da] += gear * force;
  }
  for (int d = 0; d < m.nv; ++d)
    if (m.jnt_actgravcomp[m.dof_jnt[d]]) w.qfrc_actuator[d] += w.qfrc_gravcomp[d];
}

// ------------------------------------------------------------------ FP64 operational-space control
// Symmetric Gauss-Jordan inversion without pivoting (SPD operands).  Step k: p = a_kk;
// row k <- (row k with a_kk := 1) / p; row i != k <- (row i with a_ik := 0) - a_ik * row k.
// Returns 0, or -1 when a pivot is not positive and finite.
int spd_inverse(const T* in, int n, T* a) {
  for (int k = 0; k < n * n; ++k) a[k] = in[k];
  T row[8], col[8];
  for (int k = 0; k < n; ++k) {
    T p = a[k * n + k];
    if (!(p > 0) || !std::isfinite(p)) return -1;
    for (int j = 0; j < n; ++j) row[j] = (j == k ? T(1) : a[k * n + j]) / p;
    for (int i = 0; i < n; ++i) col[i] = a[i * n + k];
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < n; ++j)
        a[i * n + j] = i == k ? row[j] : (j == k ? T(0) : a[i * n + j]) - col[i] * row[j];
  }
  return 0;
}

// One-sided Jacobi pseudo-inverse with MuJoCo-free numpy.linalg.pinv semantics (singular values
// below 1e-15 * max are dropped); restates pinv_group, gpu/cuda/control/osc_solver.cu:108-258
// (scale, cyclic column pairs, DBL_EPSILON rotation test, 64 sweeps, 2e-15 orthogonality).
int jacobi_pinv(const T* a, int n, T* out, int* rank) {
  T scale = 0;
  for (int k = 0; k < n * n; ++k) scale = std::max(scale, std::fabs(a[k]));
  for (int k = 0; k < n * n; ++k) out[k] = 0;
  *rank = 0;
  if (!(scale > 0)) return 1;
  T B[36], V[36];   // column-major: B[col*n + row]
  for (int c = 0; c < n; ++c)
    for (int r = 0; r < n; ++r) { B[c * n + r] = a[r * n + c] / scale; V[c * n + r] = r == c ? 1 : 0; }
  bool converged = false;
  for (int sweep = 0; sweep < 64; ++sweep) {
    int rotations = 0;
    for (int p = 0; p < n - 1; ++p)
      for (int q = p + 1; q < n; ++q) {
        T alpha = 0, beta = 0, gamma = 0;
        for (int r = 0; r < n; ++r) {
          alpha += B[p * n + r] * B[p * n + r];
          beta += B[q * n + r] * B[q * n + r];
          gamma += B[p * n + r] * B[q * n + r];
        }
        if (std::fabs(gamma) > 2.220446049250313e-16 * std::sqrt(alpha) * std::sqrt(beta)) {
          T zeta = (beta - alpha) / (2 * gamma);
          T t = (zeta < 0 ? -1.0 : 1.0) / (std::fabs(zeta) + std::sqrt(1 + zeta * zeta));
          T c = 1 / std::sqrt(1 + t * t), s = c * t;
          for (int r = 0; r < n; ++r) {
            T bp = B[p * n + r], bq = B[q * n + r], vp = V[p * n + r], vq = V[q * n + r];
            B[p * n + r] = c * bp - s * bq; B[q * n + r] = s * bp + c * bq;
            V[p * n + r] = c * vp - s * vq; V[q * n + r] = s * vp + c * vq;
          }
          ++rotations;
        }
      }
    if (rotations == 0) { converged = true; break; }
  }
  T norms[6], sing[6], maxnorm = 0;
  bool keep[6];
  for (int p = 0; p < n; ++p) {
    T s = 0;
    for (int r = 0; r < n; ++r) s += B[p * n + r] * B[p * n + r];
    norms[p] = s; sing[p] = std::sqrt(s); maxnorm = std::max(maxnorm, sing[p]);
  }
  int count = 0;
  for (int p = 0; p < n; ++p) { keep[p] = sing[p] > 1e-15 * maxnorm; count += keep[p]; }
  T maxcorr = 0;
  for (int p = 0; p < n; ++p)
    for (int q = p + 1; q < n; ++q)
      if (keep[p] && keep[q]) {
        T g = 0;
        for (int r = 0; r < n; ++r) g += B[p * n + r] * B[q * n + r];
        maxcorr = std::max(maxcorr, std::fabs(g) / (sing[p] * sing[q]));
      }
  if (maxcorr < 2e-15) converged = true;
  for (int r = 0; r < n; ++r)
    for (int c = 0; c < n; ++c) {
      T v = 0;
      for (int k = 0; k < n; ++k)
        if (keep[k]) v += V[k * n + r] * B[k * n + c] * ((1 / norms[k]) / scale);
      out[r * n + c] = v;
    }
  *rank = count;
  return converged ? 1 : 0;
}

// pinv of a symmetric positive semidefinite operand: the Gauss-Jordan inverse when it is provably
// the pseudo-inverse (all pivots positive and trace(A) trace(A^-1) <= 1e13 < 1e15, so no singular
// value falls under numpy's 1e-15 cutoff), else the Jacobi pseudo-inverse.  Returns ok flag.
int psd_pinv(const T* a, int n, T* out, int* rank) {
  if (spd_inverse(a, n, out) == 0) {
    T ta = 0, ti = 0;
    for (int i = 0; i < n; ++i) { ta += a[i * n + i]; ti += out[i * n + i]; }
    if (ti > 0 && ta * ti <= 1e13) { *rank = n; return 1; }
  }
  return jacobi_pinv(a, n, out, rank);
}

// robosuite OSC_POSE goal orientation: R(axis-angle delta) through robosuite's float32 quat2mat,
// as restated in rotation_delta (gpu/cuda/control/osc_solver.cu:278-306).  Exactly zero delta
// gives the identity (robosuite's axisangle2quat of a zero vector).
void rotation_delta(T x, T y, T z, T* r) {
  T angle = std::sqrt(x * x + y * y + z * z);
  if (angle == 0) {
    for (int k = 0; k < 9; ++k) r[k] = k % 4 == 0 ? 1 : 0;
    return;
  }
  T f = std::sin(angle * 0.5) / angle;
  volatile float q[4] = {(float)std::cos(angle * 0.5), (float)(x * f), (float)(y * f), (float)(z * f)};
  volatile float n = q[0] * q[0];
  n = n + q[1] * q[1];
  n = n + q[2] * q[2];
  n = n + q[3] * q[3];
  float s = (float)std::sqrt(2.0 / (double)n);
  float qs[4];
  for (int i = 0; i < 4; ++i) qs[i] = q[i] * s;
  volatile float p11 = qs[1] * qs[1], p22 = qs[2] * qs[2], p33 = qs[3] * qs[3];
  volatile float p12 = qs[1] * qs[2], p13 = qs[1] * qs[3], p23 = qs[2] * qs[3];
  volatile float p01 = qs[0] * qs[1], p02 = qs[0] * qs[2], p03 = qs[0] * qs[3];
  r[0] = (1.0 - (double)p22) - (double)p33;
  r[4] = (1.0 - (double)p11) - (double)p33;
  r[8] = (1.0 - (double)p11) - (double)p22;
  r[1] = (double)(float)(p12 - p03);
  r[2] = (double)(float)(p13 + p02);
  r[3] = (double)(float)(p12 + p03);
  r[5] = (double)(float)(p23 - p01);
  r[6] = (double)(float)(p13 - p02);
  r[7] = (double)(float)(p23 + p01);
}

// robosuite OSC_POSE (fixed impedance, delta, uncoupled pos/ori) in FP64; restates control()
// of gpu/cuda/control/osc_solver.cu:309-678 and robosuite's opspace_matrices, nullspace_torques,
// orientation_error (recipe in tests/cuda/osc_reference_fixture.py:9-33).
// n (1..8) arm joints: mass n x n, J 6 x n, q / qvel / bias / q0 / tau n, ctrlrange and ctrl for
// the n arm and two gripper actuators.
// Component k (0..5) of the pose delta: robosuite's Controller.scale_action, as the reference's
// action_component (gpu/cuda/control/osc_solver.cu:38-47).  scale null: OSC_POSE's default ranges
// (input [-1, 1], output 0.05 m / 0.5 rad); else input_min[6], input_max[6], output_min[6],
// output_max[6].
T scaled_action(const T* action, const T* scale, int k) {
  T a = action[k];
  if (!scale) return (k < 3 ? 0.05 : 0.5) * (std::isnan(a) ? a : std::min(1.0, std::max(-1.0, a)));
  T lo = scale[k], hi = scale[6 + k], olo = scale[12 + k], ohi = scale[18 + k];
  T x = std::isnan(a) ? a : std::min(hi, std::max(lo, a));
  return (x - (hi + lo) * 0.5) * (std::fabs(ohi - olo) / std::fabs(hi - lo)) + (ohi + olo) * 0.5;
}

int osc_core(int n, const T* mass, const T* J, const T* q, const T* qvel, const T* bias, const T* ee_pos,
             const T* ee_rot, const T* ee_vel, const T* action, const T* scale, const T* gains, const T* q0,
             const T* ctrlrange, int uncouple, T speed, int policy, T* goal_pos, T* goal_rot,
             T* gripper, T* tau, T* ctrl, int* rank) {
  if (n < 1 || n > 8) return MX_ERR_INVALID;
  T minv[64];
  if (spd_inverse(mass, n, minv) != 0) return MX_OSC_SINGULAR_MASS;
  T mjt[48], A[36], Ap[9], Ar[9], Lf[36], Lp[9], Lr[9], jbar[48], N[64];
  for (int i = 0; i < n; ++i)       // M^-1 J^T (n x 6)
    for (int c = 0; c < 6; ++c) {
      T s = 0;
      for (int k = 0; k < n; ++k) s += minv[i * n + k] * J[c * n + k];
      mjt[i * 6 + c] = s;
    }
  for (int r = 0; r < 6; ++r)       // A = J M^-1 J^T
    for (int c = 0; c < 6; ++c) {
      T s = 0;
      for (int k = 0; k < n; ++k) s += J[r * n + k] * mjt[k * 6 + c];
      A[r * 6 + c] = s;
    }
  for (int r = 0; r < 3; ++r)
    for (int c = 0; c < 3; ++c) { Ap[r * 3 + c] = A[r * 6 + c]; Ar[r * 3 + c] = A[(r + 3) * 6 + c + 3]; }
  int ok = psd_pinv(A, 6, Lf, rank) & psd_pinv(Ap, 3, Lp, rank + 1) & psd_pinv(Ar, 3, Lr, rank + 2);
  if (!ok) return MX_OSC_PINV_FAILED;
  for (int i = 0; i < n; ++i)       // Jbar = M^-1 J^T Lambda
    for (int c = 0; c < 6; ++c) {
      T s = 0;
      for (int k = 0; k < 6; ++k) s += mjt[i * 6 + k] * Lf[k * 6 + c];
      jbar[i * 6 + c] = s;
    }
  for (int i = 0; i < n; ++i)       // N = I - Jbar J
    for (int j = 0; j < n; ++j) {
      T s = 0;
      for (int k = 0; k < 6; ++k) s += jbar[i * 6 + k] * J[k * n + j];
      N[i * n + j] = (i == j ? 1.0 : 0.0) - s;
    }
  if (policy) {   // goal update (robosuite set_goal; reference osc_solver.cu:570-583)
    T delta[6];
    for (int k = 0; k < 6; ++k) delta[k] = scaled_action(action, scale, k);
    for (int k = 0; k < 3; ++k) goal_pos[k] = ee_pos[k] + delta[k];
    // the goal orientation moves only when some rotation component is nonzero (NaN counts)
    if (delta[3] != 0 || delta[4] != 0 || delta[5] != 0) {
      T R[9];
      rotation_delta(delta[3], delta[4], delta[5], R);
      for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
          goal_rot[3 * i + j] = R[3 * i] * ee_rot[j] + R[3 * i + 1] * ee_rot[3 + j] + R[3 * i + 2] * ee_rot[6 + j];
    }
  }
  T desired[6];
  for (int r = 0; r < 3; ++r) {
    int nx = (r + 1) % 3, ls = (r + 2) % 3;
    T er = 0;
    for (int c = 0; c < 3; ++c)
      er += 0.5 * (ee_rot[nx * 3 + c] * goal_rot[ls * 3 + c] - ee_rot[ls * 3 + c] * goal_rot[nx * 3 + c]);
    T ep = goal_pos[r] - ee_pos[r];
    desired[r] = gains[r] * ep - gains[r + 6] * ee_vel[r];
    desired[r + 3] = gains[r + 3] * er - gains[r + 9] * ee_vel[r + 3];
  }
  T wrench[6];
  if (uncouple) {
    for (int r = 0; r < 3; ++r) {
      T a = 0, b = 0;
      for (int k = 0; k < 3; ++k) { a += Lp[r * 3 + k] * desired[k]; b += Lr[r * 3 + k] * desired[3 + k]; }
      wrench[r] = a; wrench[r + 3] = b;
    }
  } else {
    for (int r = 0; r < 6; ++r) {
      T a = 0;
      for (int k = 0; k < 6; ++k) a += Lf[r * 6 + k] * desired[k];
      wrench[r] = a;
    }
  }
  T pd[8], posture[8];
  for (int c = 0; c < n; ++c) pd[c] = 10 * (q0[c] - q[c]) - 6.324555320336759 * qvel[c];
  for (int r = 0; r < n; ++r) {
    T s = 0;
    for (int k = 0; k < n; ++k) s += mass[r * n + k] * pd[k];
    posture[r] = s;
  }
  for (int i = 0; i < n; ++i) {
    T task = 0, null = 0;
    for (int k = 0; k < 6; ++k) task += J[k * n + i] * wrench[k];
    for (int k = 0; k < n; ++k) null += N[k * n + i] * posture[k];
    T t = task + bias[i] + null;
    tau[i] = t;
    ctrl[i] = std::isnan(t) ? t : std::min(ctrlrange[2 * i + 1], std::max(ctrlrange[2 * i], t));
  }
  T a6 = action[6];
  T sgn = std::isnan(a6) ? a6 : (a6 > 0 ? 1.0 : (a6 < 0 ? -1.0 : 0.0));
  for (int i = 0; i < 2; ++i) {
    T v = gripper[i] + speed * (i == 0 ? -1.0 : 1.0) * sgn;
    v = std::isnan(v) ? v : std::min(1.0, std::max(-1.0, v));
    gripper[i] = v;
    T lo = ctrlrange[2 * (i + n)], hi = ctrlrange[2 * (i + n) + 1];
    ctrl[n + i] = (hi + lo) * 0.5 + (hi - lo) * 0.5 * v;
  }
  return 0;
}

// ------------------------------------------------------------------ one world, one launch
struct Stepper {
  const OrModel& m;
  const OrData& d;
  World w;
  Stepper(const OrModel& mm, const OrData& dd) : m(mm), d(dd), w(mm) {}

  // Controller gather + OSC + scatter: fused_control_drive.cu:34-300 (gather the n x n M and 6 x n
  // J of the n = osc_ndof arm joints, q, qdot, bias, EE pose and velocity; FP64 OSC; ctrl scatter).
  void control(int world, const T* qpos, const T* qvel, T* ctrl, int policy, bool publish) {
    int nv = m.nv, on = m.osc_ndof;
    T mass[64], jac[48], q[8], qd[8], bias[8], ee_pos[3], ee_rot[9], ee_vel[6];
    site_jac(m, w, m.osc_site, w.jacp.data(), w.jacr.data());
    int t = m.dof_treeid[m.osc_dofadr[0]], n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    const T* blk = &w.M[m.tree_madr[t]];
    for (int i = 0; i < on; ++i) {
      int di = m.osc_dofadr[i];
      for (int j = 0; j < on; ++j) mass[i * on + j] = blk[(di - a) * n + (m.osc_dofadr[j] - a)];
      for (int k = 0; k < 3; ++k) {
        jac[k * on + i] = w.jacp[k * nv + di];
        jac[(k + 3) * on + i] = w.jacr[k * nv + di];
      }
      q[i] = qpos[m.osc_qposadr[i]];
      qd[i] = qvel[di];
      bias[i] = w.qfrc_bias[di];
    }
    for (int k = 0; k < 3; ++k) ee_pos[k] = w.site_xpos[3 * m.osc_site + k];
    for (int k = 0; k < 9; ++k) ee_rot[k] = w.site_xmat[9 * m.osc_site + k];
    for (int k = 0; k < 3; ++k) {
      T vp = 0, vr = 0;
      for (int i = 0; i < nv; ++i) { vp += w.jacp[k * nv + i] * qvel[i]; vr += w.jacr[k * nv + i] * qvel[i]; }
      ee_vel[k] = vp; ee_vel[k + 3] = vr;
    }
    if (publish) {
      std::copy(mass, mass + on * on, d.osc_mass + on * on * world);
      std::copy(jac, jac + 6 * on, d.osc_jac + 6 * on * world);
      std::copy(q, q + on, d.osc_q + on * world);
      std::copy(qd, qd + on, d.osc_qvel + on * world);
      std::copy(bias, bias + on, d.osc_bias + on * world);
      std::copy(ee_pos, ee_pos + 3, d.osc_ee_pos + 3 * world);
      std::copy(ee_rot, ee_rot + 9, d.osc_ee_rot + 9 * world);
      std::copy(ee_vel, ee_vel + 6, d.osc_ee_vel + 6 * world);
    }
    if (d.osc_error[world] != 0) return;
    T range[20], tau[8], c[10];
    for (int i = 0; i < on + 2; ++i) {
      range[2 * i] = m.actuator_ctrlrange[2 * m.osc_actuator[i]];
      range[2 * i + 1] = m.actuator_ctrlrange[2 * m.osc_actuator[i] + 1];
    }
    int err = osc_core(on, mass, jac, q, qd, bias, ee_pos, ee_rot, ee_vel, d.osc_action + 7 * world,
                       m.osc_action_scaled ? d.osc_action_scale + MX_OSC_ACTION_SCALE * world : nullptr,
                       d.osc_gains + 12 * world, d.osc_q0 + on * world, range, m.osc_uncouple,
                       m.osc_gripper_speed, policy, d.osc_goal_pos + 3 * world, d.osc_goal_rot + 9 * world,
                       d.osc_gripper + 2 * world, tau, c, d.osc_rank + 3 * world);
    if (err) { d.osc_error[world] = err; return; }
    std::copy(tau, tau + on, d.osc_tau + on * world);
    for (int i = 0; i < on + 2; ++i) ctrl[m.osc_actuator[i]] = c[i];
  }

  // One substep (or a forward pass): step1 -> OSC -> solve -> integrate, the schedule of
  // Runtime.enqueue_substep (gpu/host/backends/cuda_fp32/runtime.py:40-45).
  void substep(int world, T* qpos, T* qvel, T* ctrl, T* warm, T* time, int policy, int flags, bool last) {
    int nv = m.nv;
    kinematics(m, qpos, w);
    com_pos(m, w);
    crb(m, w);
    factor(m, w.M.data(), w.L.data(), nullptr, 0);
    collision(m, w, m.has_body_active ? d.body_active + (size_t)m.nbody * world : nullptr);
    make_constraint(m, w, qpos, qvel);
    com_vel(m, qvel, w);
    rne(m, qvel, w);
    passive(m, qpos, qvel, w);
    gravcomp(m, w);
    fluid(m, qvel, w);
    const T* xfrc = d.xfrc_applied + (size_t)6 * m.nbody * world;
    xfrc_project(m, xfrc, w);
    if (flags & MX_FLAG_BOOTSTRAP) {
      for (int k = 0; k < 3; ++k) d.osc_goal_pos[3 * world + k] = w.site_xpos[3 * m.osc_site + k];
      for (int k = 0; k < 9; ++k) d.osc_goal_rot[9 * world + k] = w.site_xmat[9 * m.osc_site + k];
      d.osc_gripper[2 * world] = d.osc_gripper[2 * world + 1] = 0;
      d.osc_error[world] = 0;
    }
    if (!(flags & MX_FLAG_NO_CONTROL)) control(world, qpos, qvel, ctrl, policy, last);
    actuation(m, qpos, qvel, ctrl, w);
    const T* applied = d.qfrc_applied + (size_t)nv * world;
    for (int i = 0; i < nv; ++i)
      w.qfrc_smooth[i] = w.qfrc_passive[i] - w.qfrc_bias[i] + applied[i] + w.qfrc_actuator[i] + w.qfrc_xfrc[i];
    std::copy(w.qfrc_smooth.begin(), w.qfrc_smooth.end(), w.qacc_smooth.begin());
    solve(m, w.L.data(), w.qacc_smooth.data());
    newton(m, w, warm);
    if (m.njmax > 0) {   // rows, contacts and Newton iterations summed over substeps until cleared
      T* st = d.stat_sums + 4 * (size_t)world;
      st[0] += w.nefc;
      st[1] += std::min((int)w.contacts.size(), m.nconmax);
      st[2] += w.niter;
      st[3] += (T)w.niter * w.nefc;
    }
    if (last) {
      post_constraint(m, qvel, xfrc, w, d.sensordata + (size_t)m.nsensordata * world);
      publish(world, ctrl);
    }
    if (flags & MX_FLAG_NO_INTEGRATE) return;
    euler(world, qpos, qvel, warm, time);
  }

  // Semi-implicit Euler with implicit joint damping: MuJoCo mj_Euler; reference
  // gpu/cuda/fp32/fused_euler_step.cu:35-269 and fused_tail.cu:15-90 (advance).
  void euler(int world, T* qpos, T* qvel, T* warm, T* time) {
    int nv = m.nv;
    T h = m.opt_timestep;
    bool damped = false;
    if (!(m.opt_disableflags & (1 << 15)))
      for (int i = 0; i < nv; ++i) damped |= m.dof_damping[i] > 0;
    std::vector<T>& acc = w.tmp;
    for (int i = 0; i < nv; ++i) acc[i] = w.qacc[i];
    if (damped) {
      factor(m, w.M.data(), w.L2.data(), m.dof_damping, h);
      for (int i = 0; i < nv; ++i) acc[i] = w.qfrc_smooth[i] + w.qfrc_constraint[i];
      solve(m, w.L2.data(), acc.data());
    }
    for (int i = 0; i < nv; ++i) warm[i] = w.qacc[i];
    for (int i = 0; i < nv; ++i) qvel[i] += h * acc[i];
    for (int j = 0; j < m.njnt; ++j) {
      int qa = m.jnt_qposadr[j], da = m.jnt_dofadr[j];
      if (m.jnt_type[j] == 0) {
        for (int k = 0; k < 3; ++k) qpos[qa + k] += h * qvel[da + k];
        T* quat = qpos + qa + 3;
        T v[3] = {qvel[da + 3], qvel[da + 4], qvel[da + 5]};
        T nrm = std::sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
        T axis[3] = {1, 0, 0}, angle = 0;
        if (nrm >= kMinVal) { for (int k = 0; k < 3; ++k) axis[k] = v[k] / nrm; angle = h * nrm; }
        T qr[4] = {std::cos(angle / 2), axis[0] * std::sin(angle / 2), axis[1] * std::sin(angle / 2),
                   axis[2] * std::sin(angle / 2)};
        normalize4(quat);
        T out[4];
        qmul(quat, qr, out);
        for (int k = 0; k < 4; ++k) quat[k] = out[k];
      } else if (m.jnt_type[j] == 2 || m.jnt_type[j] == 3) {
        qpos[qa] += h * qvel[da];
      }
    }
    *time += h;
    d.nstep[world] += 1;
  }

  void publish(int world, const T* ctrl) {
    int nv = m.nv, nb = m.nbody;
    auto put = [&](T* dst, const std::vector<T>& src, size_t width) {
      std::copy(src.begin(), src.begin() + width, dst + width * world);
    };
    put(d.qacc, w.qacc, nv); put(d.qacc_smooth, w.qacc_smooth, nv); put(d.qfrc_bias, w.qfrc_bias, nv);
    put(d.qfrc_passive, w.qfrc_passive, nv); put(d.qfrc_actuator, w.qfrc_actuator, nv);
    put(d.qfrc_smooth, w.qfrc_smooth, nv); put(d.qfrc_constraint, w.qfrc_constraint, nv);
    put(d.actuator_force, w.actuator_force, m.nu); put(d.M, w.M, m.nM);
    put(d.xpos, w.xpos, 3 * nb); put(d.xquat, w.xquat, 4 * nb); put(d.xmat, w.xmat, 9 * nb);
    put(d.geom_xpos, w.geom_xpos, 3 * m.ngeom); put(d.geom_xmat, w.geom_xmat, 9 * m.ngeom);
    put(d.site_xpos, w.site_xpos, 3 * m.nsite); put(d.site_xmat, w.site_xmat, 9 * m.nsite);
    put(d.subtree_com, w.subtree_com, 3 * nb);
    put(d.cacc, w.cacc_post, 6 * nb); put(d.cfrc_int, w.cfrc_int, 6 * nb); put(d.cfrc_ext, w.cfrc_ext, 6 * nb);
    (void)ctrl;
    int C = m.nconmax, R = m.njmax;
    int ncon = std::min((int)w.contacts.size(), C);
    d.ncon[world] = ncon;
    for (int c = 0; c < ncon; ++c) {
      const Contact& ct = w.contacts[c];
      size_t b = (size_t)C * world + c;
      for (int k = 0; k < 3; ++k) d.contact_pos[3 * b + k] = ct.pos[k];
      for (int k = 0; k < 9; ++k) d.contact_frame[9 * b + k] = ct.frame[k];
      for (int k = 0; k < 5; ++k) d.contact_friction[5 * b + k] = ct.friction[k];
      d.contact_dist[b] = ct.dist;
      d.contact_includemargin[b] = ct.includemargin;
      d.contact_geom[2 * b] = ct.geom[0];
      d.contact_geom[2 * b + 1] = ct.geom[1];
      d.contact_dim[b] = ct.dim;
    }
    d.nefc[world] = w.nefc;
    for (int r = 0; r < w.nefc && r < R; ++r) {
      size_t b = (size_t)R * world + r;
      d.efc_force[b] = w.force[r];
      d.efc_pos[b] = w.efc_pos[r];
      d.efc_D[b] = w.D[r];
      d.efc_aref[b] = w.aref[r];
      d.efc_type[b] = w.type[r];
      d.efc_state[b] = w.state[r];
      d.efc_id[b] = w.id[r];
    }
    d.solver_niter[world] = w.niter;
    // capacity and failure bits stay set until the caller clears them; the iteration-limit bits
    // describe the last substep only (as the device library)
    const int last = MX_OVERFLOW_ITERATIONS | MX_OVERFLOW_LS_ITERATIONS;
    d.overflow[world] = (d.overflow[world] & ~last) | w.overflow;
  }

  void run(int world, int substeps, int flags) {
    int nq = m.nq, nv = m.nv, nu = m.nu;
    T* qpos = d.qpos + (size_t)nq * world;
    T* qvel = d.qvel + (size_t)nv * world;
    T* ctrl = d.ctrl + (size_t)nu * world;
    T* warm = d.qacc_warmstart + (size_t)nv * world;
    T* time = d.time + world;
    for (int s = 0; s < substeps; ++s) {
      int policy = (flags & MX_FLAG_POLICY_FIRST) && s == 0;
      int f = flags & ~(s > 0 ? MX_FLAG_BOOTSTRAP : 0);
      substep(world, qpos, qvel, ctrl, warm, time, policy, f, s == substeps - 1);
    }
  }
};

void pin_thread(int core) {
  cpu_set_t set;
  CPU_ZERO(&set);
  CPU_SET(core, &set);
  sched_setaffinity(0, sizeof set, &set);
}

template <class F>
void parallel_worlds(int nworld, int threads, int pin, F&& body) {
  threads = std::max(1, std::min(threads, nworld));
  if (threads == 1) {
    for (int w = 0; w < nworld; ++w) body(w);
    return;
  }
  std::atomic<int> next(0);
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t)
    pool.emplace_back([&, t]() {
      if (pin) pin_thread(t % (int)std::thread::hardware_concurrency());
      for (int w = next++; w < nworld; w = next++) body(w);
    });
  for (auto& th : pool) th.join();
}

const char* field_name(int which, int index) {
  static const char* model_real[] = {
#define N(name) #name,
      MX_MODEL_REAL_ARRAYS(N)};
  static const char* model_int[] = {MX_MODEL_INT_ARRAYS(N)};
  static const char* model_iscal[] = {MX_MODEL_INT_SCALARS(N)};
  static const char* model_rscal[] = {MX_MODEL_REAL_SCALARS(N)};
  static const char* data_real[] = {MX_DATA_REAL_ARRAYS(N)};
  static const char* data_f64[] = {MX_DATA_F64_ARRAYS(N)};
  static const char* data_int[] = {MX_DATA_INT_ARRAYS(N)};
#undef N
  const char** tables[] = {model_real, model_int, model_iscal, model_rscal, data_real, data_f64, data_int};
  const int counts[] = {int(sizeof model_real / sizeof(char*)), int(sizeof model_int / sizeof(char*)),
                        int(sizeof model_iscal / sizeof(char*)), int(sizeof model_rscal / sizeof(char*)),
                        int(sizeof data_real / sizeof(char*)), int(sizeof data_f64 / sizeof(char*)),
                        int(sizeof data_int / sizeof(char*))};
  if (which < 0 || which > 6) return nullptr;
  if (index == -1) return reinterpret_cast<const char*>(static_cast<intptr_t>(counts[which]));
  if (index < 0 || index >= counts[which]) return nullptr;
  return tables[which][index];
}

}  // namespace orc

using namespace orc;

extern "C" {
size_t or_model_bytes(void) { return sizeof(OrModel); }
size_t or_data_bytes(void) { return sizeof(OrData); }
int or_field_count(int which) { return (int)reinterpret_cast<intptr_t>(field_name(which, -1)); }
const char* or_field_name(int which, int index) { return index < 0 ? nullptr : field_name(which, index); }

int or_control_step(const OrModel* m, const OrData* d, int substeps, int flags, int threads, int pin) {
  if (!m || !d || substeps < 0 || d->nworld < 1 || m->abi_version != MX_ABI_VERSION) return MX_ERR_INVALID;
  parallel_worlds(d->nworld, threads, pin, [&](int w) {
    thread_local std::vector<char> dummy;
    Stepper s(*m, *d);
    s.run(w, substeps, flags);
  });
  return 0;
}

int or_forward(const OrModel* m, const OrData* d, const int32_t* mask, int flags, int threads) {
  if (!m || !d || d->nworld < 1 || m->abi_version != MX_ABI_VERSION) return MX_ERR_INVALID;
  parallel_worlds(d->nworld, threads, 0, [&](int w) {
    if (mask && !mask[w]) return;
    Stepper s(*m, *d);
    s.run(w, 1, (flags | MX_FLAG_NO_INTEGRATE) & ~MX_FLAG_POLICY_FIRST);
  });
  return 0;
}

int or_osc(int ndof, const double* mass, const double* jac, const double* q, const double* qvel, const double* bias,
           const double* ee_pos, const double* ee_rot, const double* ee_vel, const double* action,
           const double* action_scale, const double* gains, const double* q0, const double* ctrlrange, int uncouple,
           double gripper_speed, int policy, double* goal_pos, double* goal_rot, double* gripper,
           double* tau, double* ctrl, int32_t* rank) {
  int r[3] = {0, 0, 0};
  int err = osc_core(ndof, mass, jac, q, qvel, bias, ee_pos, ee_rot, ee_vel, action, action_scale, gains, q0, ctrlrange,
                     uncouple, gripper_speed, policy, goal_pos, goal_rot, gripper, tau, ctrl, r);
  for (int k = 0; k < 3; ++k) rank[k] = r[k];
  return err;
}

int or_spd_inverse(const double* a, int n, double* out) {
  if (n < 1 || n > 8) return MX_ERR_INVALID;
  return spd_inverse(a, n, out);
}

int or_pinv(const double* a, int n, double* out, int32_t* rank) {
  if (n < 1 || n > 6) return MX_ERR_INVALID;
  int r = 0;
  int ok = psd_pinv(a, n, out, &r);
  *rank = r;
  return ok;
}
}
