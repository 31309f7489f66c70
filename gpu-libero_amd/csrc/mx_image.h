// Model image: the model arrays re-packed, once per launch, into per-entity records in LDS.
//
// Every wavefront (world) copies the read-only model from HBM into its LDS at kernel entry, so the
// substep loop reads model data with LDS latency instead of dependent global loads.  Records mix
// int and float fields in 32-bit words; record strides are odd so that lanes reading one field of
// consecutive entities hit distinct LDS banks.
#pragma once
#include <hip/hip_runtime.h>
#include "../../include/mx_physics.h"

namespace MX_NS {

// The model as the kernels see it: read in place in the kernel argument segment (address space 4,
// constant memory read with scalar loads).
typedef const __attribute__((address_space(4))) MxModel KModel;

// body record
constexpr int BR = 31;
enum : int { B_PARENT, B_ROOT, B_WELD, B_TREE, B_JNTADR, B_JNTNUM, B_DOFADR, B_DOFNUM, B_SUBTREE, B_LASTDOF,
             B_POS = 10, B_QUAT = 13, B_IPOS = 17, B_IQUAT = 20, B_MASS = 24, B_SMASS = 25, B_INERTIA = 26,
             B_INVW = 29 };
// joint record
constexpr int JR = 25;
enum : int { J_TYPE, J_BODY, J_QPOS, J_DOF, J_LIMITED, J_POS = 5, J_AXIS = 8, J_RANGE = 11, J_STIFF = 13,
             J_MARGIN = 14, J_SOLREF = 15, J_SOLIMP = 17, J_QPOS0 = 22, J_SPRING = 23 };
// dof record
constexpr int DR = 15;
enum : int { D_BODY, D_JNT, D_PARENT, D_TREE, D_ARM = 4, D_DAMP = 5, D_FLOSS = 6, D_INVW = 7, D_SOLREF = 8,
             D_SOLIMP = 10 };
// geom record
constexpr int GR = 37;
enum : int { G_TYPE, G_BODY, G_CONTYPE, G_CONAFF, G_CONDIM, G_PRIORITY, G_DATAID, G_POS = 7, G_QUAT = 10,
             G_SIZE = 14, G_RBOUND = 17, G_AABB = 18, G_FRIC = 24, G_SOLREF = 27, G_SOLIMP = 29, G_SOLMIX = 34,
             G_MARGIN = 35, G_GAP = 36 };
// site record
constexpr int SR = 9;
enum : int { S_BODY, S_POS = 1, S_QUAT = 4 };
// actuator record (A_QPOS, A_DOF: the transmission joint's qpos and dof addresses)
constexpr int AR = 15;
enum : int { A_TRN, A_BIAS, A_CTRLLIM, A_FORCELIM, A_GEAR = 4, A_GAIN = 5, A_BIASPRM = 6, A_CTRLRANGE = 9,
             A_FORCERANGE = 11, A_QPOS = 13, A_DOF = 14 };
// tree record: dof address, dof count, mass-block address, damped-block address (after the nM mass
// entries; -1: the tree has no joint damping)
constexpr int TR = 4;
enum : int { T_DOFADR, T_DOFNUM, T_MADR, T_DAMPADR };

// Word offsets of each record group in the image.
struct Image {
  int body, jnt, dof, geom, site, act, tree, mpair, mentry, level, osc, chain, chainw, pair, mesh, meshrec, words;
};

__host__ __device__ inline int img_round(int x) { return (x + 3) & ~3; }

__host__ __device__ inline Image image_layout(const MxModel& m) {
  Image I{};
  int at = 0;
  I.body = at; at += img_round(BR * m.nbody);
  I.jnt = at; at += img_round(JR * m.njnt);
  I.dof = at; at += img_round(DR * m.nv);
  I.geom = at; at += img_round(GR * m.ngeom);
  I.site = at; at += img_round(SR * m.nsite);
  I.act = at; at += img_round(AR * m.nu);
  I.tree = at; at += img_round(TR * m.ntree);
  I.mpair = at; at += img_round(2 * m.nMpair);
  I.mentry = at; at += img_round(2 * (m.nM + m.nMdamp));
  I.level = at; at += img_round(m.nlevel + 1 + m.nbody);
  I.osc = at; at += img_round(3 * MX_OSC_MAXDOF + 2);   // qpos and dof addresses, then the actuators
  // per body: number of dofs on the path world..body, then those dofs (body first, root last)
  I.chainw = m.maxchain + 1;
  I.chain = at; at += img_round(I.chainw * m.nbody);
  I.pair = at; at += img_round(m.njmax > 0 ? 2 * m.npair : 0);
  I.mesh = at; at += img_round(m.njmax > 0 ? 4 * m.nmeshvert : 0);   // x, y, z, pad: one 16-byte LDS read
  I.meshrec = at; at += img_round(m.njmax > 0 ? 2 * m.nmesh : 0);
  I.words = at;
  return I;
}

// Copy the model arrays into the image (all lanes of the wavefront cooperate).
// m and I are read in place in the kernel argument segment.
__device__ inline void stage_image(KModel& m, const __attribute__((address_space(4))) Image& I, float* f, int lane,
                                   int lanes) {
  int* n = reinterpret_cast<int*>(f);
  for (int t = lane; t < m.nbody * BR; t += lanes) {
    int b = t / BR, k = t % BR;
    float* rf = f + I.body + BR * b;
    int* ri = n + I.body + BR * b;
    switch (k) {
      case B_PARENT: ri[k] = m.body_parent[b]; break;
      case B_ROOT: ri[k] = m.body_rootid[b]; break;
      case B_WELD: ri[k] = m.body_weldid[b]; break;
      case B_TREE: ri[k] = m.body_treeid[b]; break;
      case B_JNTADR: ri[k] = m.body_jntadr[b]; break;
      case B_JNTNUM: ri[k] = m.body_jntnum[b]; break;
      case B_DOFADR: ri[k] = m.body_dofadr[b]; break;
      case B_DOFNUM: ri[k] = m.body_dofnum[b]; break;
      case B_SUBTREE: ri[k] = m.body_subtreesize[b]; break;
      case B_LASTDOF: ri[k] = m.body_lastdof[b]; break;
      case B_MASS: rf[k] = m.body_mass[b]; break;
      case B_SMASS: rf[k] = m.body_subtreemass[b]; break;
      default:
        if (k < B_QUAT) rf[k] = m.body_pos[3 * b + k - B_POS];
        else if (k < B_IPOS) rf[k] = m.body_quat[4 * b + k - B_QUAT];
        else if (k < B_IQUAT) rf[k] = m.body_ipos[3 * b + k - B_IPOS];
        else if (k < B_MASS) rf[k] = m.body_iquat[4 * b + k - B_IQUAT];
        else if (k < B_INVW) rf[k] = m.body_inertia[3 * b + k - B_INERTIA];
        else rf[k] = m.body_invweight0[2 * b + k - B_INVW];
    }
  }
  for (int t = lane; t < m.njnt * JR; t += lanes) {
    int j = t / JR, k = t % JR;
    float* rf = f + I.jnt + JR * j;
    int* ri = n + I.jnt + JR * j;
    int qa = m.jnt_qposadr[j];
    switch (k) {
      case J_TYPE: ri[k] = m.jnt_type[j]; break;
      case J_BODY: ri[k] = m.jnt_body[j]; break;
      case J_QPOS: ri[k] = qa; break;
      case J_DOF: ri[k] = m.jnt_dofadr[j]; break;
      case J_LIMITED: ri[k] = m.jnt_limited[j]; break;
      case J_STIFF: rf[k] = m.jnt_stiffness[j]; break;
      case J_MARGIN: rf[k] = m.jnt_margin[j]; break;
      case J_QPOS0: rf[k] = m.jnt_type[j] == 0 ? 0.f : m.qpos0[qa]; break;
      case J_SPRING: rf[k] = m.jnt_type[j] == 0 ? 0.f : m.qpos_spring[qa]; break;
      default:
        if (k < J_AXIS) rf[k] = m.jnt_pos[3 * j + k - J_POS];
        else if (k < J_RANGE) rf[k] = m.jnt_axis[3 * j + k - J_AXIS];
        else if (k < J_STIFF) rf[k] = m.jnt_range[2 * j + k - J_RANGE];
        else if (k < J_SOLIMP) rf[k] = m.jnt_solref[2 * j + k - J_SOLREF];
        else rf[k] = m.jnt_solimp[5 * j + k - J_SOLIMP];
    }
  }
  for (int t = lane; t < m.nv * DR; t += lanes) {
    int d = t / DR, k = t % DR;
    float* rf = f + I.dof + DR * d;
    int* ri = n + I.dof + DR * d;
    switch (k) {
      case D_BODY: ri[k] = m.dof_body[d]; break;
      case D_JNT: ri[k] = m.dof_jnt[d]; break;
      case D_PARENT: ri[k] = m.dof_parent[d]; break;
      case D_TREE: ri[k] = m.dof_treeid[d]; break;
      case D_ARM: rf[k] = m.dof_armature[d]; break;
      case D_DAMP: rf[k] = m.dof_damping[d]; break;
      case D_FLOSS: rf[k] = m.dof_frictionloss[d]; break;
      case D_INVW: rf[k] = m.dof_invweight0[d]; break;
      default:
        if (k < D_SOLIMP) rf[k] = m.dof_solref[2 * d + k - D_SOLREF];
        else rf[k] = m.dof_solimp[5 * d + k - D_SOLIMP];
    }
  }
  for (int t = lane; t < m.ngeom * GR; t += lanes) {
    int g = t / GR, k = t % GR;
    float* rf = f + I.geom + GR * g;
    int* ri = n + I.geom + GR * g;
    switch (k) {
      case G_TYPE: ri[k] = m.geom_type[g]; break;
      case G_BODY: ri[k] = m.geom_body[g]; break;
      case G_CONTYPE: ri[k] = m.geom_contype[g]; break;
      case G_CONAFF: ri[k] = m.geom_conaffinity[g]; break;
      case G_CONDIM: ri[k] = m.geom_condim[g]; break;
      case G_PRIORITY: ri[k] = m.geom_priority[g]; break;
      case G_DATAID: ri[k] = m.geom_dataid[g]; break;
      case G_RBOUND: rf[k] = m.geom_rbound[g]; break;
      case G_SOLMIX: rf[k] = m.geom_solmix[g]; break;
      case G_MARGIN: rf[k] = m.geom_margin[g]; break;
      case G_GAP: rf[k] = m.geom_gap[g]; break;
      default:
        if (k < G_QUAT) rf[k] = m.geom_pos[3 * g + k - G_POS];
        else if (k < G_SIZE) rf[k] = m.geom_quat[4 * g + k - G_QUAT];
        else if (k < G_RBOUND) rf[k] = m.geom_size[3 * g + k - G_SIZE];
        else if (k < G_FRIC) rf[k] = m.geom_aabb[6 * g + k - G_AABB];
        else if (k < G_SOLREF) rf[k] = m.geom_friction[3 * g + k - G_FRIC];
        else if (k < G_SOLIMP) rf[k] = m.geom_solref[2 * g + k - G_SOLREF];
        else rf[k] = m.geom_solimp[5 * g + k - G_SOLIMP];
    }
  }
  for (int t = lane; t < m.nsite * SR; t += lanes) {
    int s = t / SR, k = t % SR;
    if (k == S_BODY) n[I.site + SR * s + k] = m.site_body[s];
    else if (k < S_QUAT) f[I.site + SR * s + k] = m.site_pos[3 * s + k - S_POS];
    else f[I.site + SR * s + k] = m.site_quat[4 * s + k - S_QUAT];
  }
  for (int t = lane; t < m.nu * AR; t += lanes) {
    int a = t / AR, k = t % AR;
    float* rf = f + I.act + AR * a;
    int* ri = n + I.act + AR * a;
    switch (k) {
      case A_TRN: ri[k] = m.actuator_trnid[a]; break;
      case A_BIAS: ri[k] = m.actuator_biastype[a]; break;
      case A_CTRLLIM: ri[k] = m.actuator_ctrllimited[a]; break;
      case A_FORCELIM: ri[k] = m.actuator_forcelimited[a]; break;
      case A_GEAR: rf[k] = m.actuator_gear[a]; break;
      case A_GAIN: rf[k] = m.actuator_gainprm[a]; break;
      case A_QPOS: ri[k] = m.jnt_qposadr[m.actuator_trnid[a]]; break;
      case A_DOF: ri[k] = m.jnt_dofadr[m.actuator_trnid[a]]; break;
      default:
        if (k < A_CTRLRANGE) rf[k] = m.actuator_biasprm[3 * a + k - A_BIASPRM];
        else if (k < A_FORCERANGE) rf[k] = m.actuator_ctrlrange[2 * a + k - A_CTRLRANGE];
        else rf[k] = m.actuator_forcerange[2 * a + k - A_FORCERANGE];
    }
  }
  for (int t = lane; t < m.ntree * TR; t += lanes) {
    int tr = t / TR, k = t % TR;
    n[I.tree + t] = k == T_DOFADR ? m.tree_dofadr[tr] : (k == T_DOFNUM ? m.tree_dofnum[tr] :
                    (k == T_MADR ? m.tree_madr[tr] : (m.tree_dampadr[tr] < 0 ? -1 : m.nM + m.tree_dampadr[tr])));
  }
  for (int t = lane; t < m.nMpair; t += lanes) {
    n[I.mpair + 2 * t] = m.mpair_i[t];
    n[I.mpair + 2 * t + 1] = m.mpair_j[t];
  }
  // mass-block entry -> block address (10 bits), size (6), row (6), column (6); then the row's dof.
  // The damped blocks of damped trees follow the nM mass entries.
  for (int tr = 0; tr < m.ntree; ++tr) {
    int nn = m.tree_dofnum[tr];
    for (int pass = 0; pass < 2; ++pass) {
      if (pass == 1 && m.tree_dampadr[tr] < 0) break;
      int adr = pass == 0 ? m.tree_madr[tr] : m.nM + m.tree_dampadr[tr];
      for (int e = lane; e < nn * nn; e += lanes) {
        n[I.mentry + 2 * (adr + e)] = adr | (nn << 10) | ((e / nn) << 16) | ((e % nn) << 22);
        n[I.mentry + 2 * (adr + e) + 1] = m.tree_dofadr[tr] + e / nn;
      }
    }
  }
  for (int b = lane; b < m.nbody; b += lanes) {
    int* ch = n + I.chain + I.chainw * b;
    int cnt = 0;
    for (int dd = m.body_lastdof[b]; dd >= 0; dd = m.dof_parent[dd]) ch[1 + cnt++] = dd;
    ch[0] = cnt;
  }
  for (int t = lane; t < m.nlevel + 1; t += lanes) n[I.level + t] = m.level_adr[t];
  for (int t = lane; t < m.nbody - 1; t += lanes) n[I.level + m.nlevel + 1 + t] = m.level_body[t];
  if (lane < m.osc_ndof) {
    n[I.osc + lane] = m.osc_qposadr[lane];
    n[I.osc + MX_OSC_MAXDOF + lane] = m.osc_dofadr[lane];
  }
  if (lane < m.osc_ndof + 2) n[I.osc + 2 * MX_OSC_MAXDOF + lane] = m.osc_actuator[lane];
  if (m.njmax > 0) {
    for (int t = lane; t < 2 * m.npair; t += lanes) n[I.pair + t] = m.pair_geom[t];
    for (int t = lane; t < 4 * m.nmeshvert; t += lanes) f[I.mesh + t] = (t & 3) == 3 ? 0.f : m.mesh_vert[3 * (t >> 2) + (t & 3)];
    for (int t = lane; t < m.nmesh; t += lanes) {
      n[I.meshrec + 2 * t] = m.mesh_vertadr[t];
      n[I.meshrec + 2 * t + 1] = m.mesh_vertnum[t];
    }
  }
}

}  // namespace mx
