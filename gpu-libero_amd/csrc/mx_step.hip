// World-local control-step kernel for gfx950 (MI355X) and the C ABI of libmx_physics.so.
//
// One 64-lane wavefront owns one world for a whole control step, following the reference schedule
// step1 -> OSC -> solve -> integrate (gpu/host/backends/cuda_fp32/runtime.py:40-45,
// physics.py:585-633).  At entry it stages the world's state into its working set; the world's
// fields in HBM are read at entry and written at exit (state, controller state and, from the last
// substep, the derived fields).  The working set and the model (as per-entity records,
// mx_image.h) live in LDS (this file's default build), or, built with MX_SLAB (mx_step_slab.hip),
// in a per-world slab of a caller-given workspace with the model image in slab 0 and a per-world
// LDS window that each stage uses for its own temporaries.
//
// Provenance: the constraint impedance and row formulas (impedance, publish_row) and the exact line
// search's per-row cost (cone_quadratic_shifted, eval_shifted) restate reference files headed
// "Copyright 2025 The Newton Developers, SPDX-License-Identifier: Apache-2.0"
// (gpu/cuda/dynamics/mjwarp_constraint_build.cu, gpu/cuda/newton/mjwarp_linesearch.cu).
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstring>
#include <cmath>
#include <mutex>
#include "../../include/mx_physics.h"
#include "mx_math.h"
#include "mx_image.h"
#include "mx_collide.h"
#include "mx_convex.h"
#include "mx_observe.h"

namespace MX_NS {

constexpr int kLanes = 64;

// Offsets of the per-world LDS arena: the model image first, then world floats (offsets in
// floats from the start), then doubles (offsets in doubles from `dbase`, a byte offset).
struct Layout {
  int img;
  int qpos, qvel, ctrl, warm, applied, xpos, xquat, xmat, xipos, ximat, xanchor, xaxis, scom, cinert, crb;
  int cdof, cvel, cdofdot, cfrcb, cfrc, M, Minv, gj0, gj1, gxpos, gxmat, sxpos, sxmat, bias, passive, act, smooth;
  int qacc_smooth, qacc, qcon, tmp, rhs, actforce, jacp, jacr, misc;
  int tp0, tq0, tp1, tq1, anc0, anc1, jl;
  int xfrc, cacc, cext, gcomp, xq;    // applied body wrenches, post-constraint, gravity compensation
  // contacts, contact-space Jacobians, constraint rows, islands, Newton workspace
  int cand, sv, bact;
  int cpos, cframe, cdist, cfric, csolref, csolimp, cmargin, cgeom, cdim, caddr, cjidx, cjval, cjn, cdot;
  int rid, rD, raref, rjaref, rjv, rforce, rstate, rquad;
  int tisl, toff, disl, dloc, iblk, isz, idof, istart, H, colk, Ma, grad, search, Mv;
  int epa, epa_req, epa_vc, epa_fc;   // EPA polytope and request block (alias the rows during collision)
  int epa_ng, epa_gw, epa_svc, epa_sfc;   // workspace route: row-group EPA blocks (count, words, capacities)
  int stage;                          // workspace route: contact staging in the LDS window (-1: none)
  int gpose;                          // workspace route: the geoms' collision records in the LDS window
  int meshw;                          // workspace route: the hull vertices' copy in the LDS window
  int hmap, cjmap;                    // workspace route: Hessian targets of M entries and Jacobian columns
  int cq, cqn;                        // workspace route: per-contact Hessian weights (doubles) and column counts
  int hown;                           // workspace route: the sweep's per-lane entry decodes (kSweepWords x 64)
  int ctrp;                           // workspace route: the contact trees the island tables were built for
  int win;                            // workspace route: words of the per-world LDS window
  int nfloat, dbase;
  int m7, minv, J, mjt, A, Ap, Ar, Lf, Lp, Lr, jbar, N, q, qd, dbias, eepos, eerot, eevel;
  int goalpos, goalrot, grip, R, desired, wrench, pd, posture, tau, action, gains, q0, work, ndouble;
  int otmp, otmp_end;                 // the controller's per-substep temporaries (doubles)
  int bytes;
};

inline int round_up(int x, int a) { return (x + a - 1) / a * a; }

constexpr int kEpaRequest = 48;   // words of the EPA request block after the polytope
// Workspace route: capacities of the small polytopes that four 16-lane rows expand at once (nine
// expansion steps' vertices, about seven steps' faces; a pair that outgrows one is expanded again
// by the whole wave on the full-size polytope)
constexpr int kSmallPolyVerts = 14, kSmallPolyFaces = 40;
// Workspace route: words of the contact staging's per-pair record (material, geoms, condim, the
// second frame axis) and per-contact record (point, normal, distance, owner lane and index)
constexpr int kStagePair = 18, kStageContact = 8;
// Workspace route: 4-byte words of LDS per world for the stages' temporaries (mass-matrix inverse,
// collision records, EPA polytope, controller, Newton's contact Jacobian and Hessian blocks).
// With the scalar slots after it a world takes exactly 10 KB, so sixteen worlds fill the CU's
// 160 KB.
constexpr int kWindowWords = 2512;
constexpr int kLdsScalars = 48;
// workspace route: per-geom collision record in the LDS window during the collision stage (pose,
// size, type, margin, gap, bounding radius, hull vertices: image word offset and count)
enum : int { GP_POS = 0, GP_MAT = 3, GP_SIZE = 12, GP_TYPE = 15, GP_MARGIN = 16, GP_GAP = 17, GP_RBOUND = 18,
             GP_VERT = 19, GP_NVERT = 20, GP_WORDS = 21 };     // workspace route: the misc and sv slots, in LDS after the window
// Island sweep: block entries whose (island, row, column) a lane keeps in registers, and the words
// per lane of the workspace route's per-substep cache of those decodes (3 per entry + 4).  The
// workspace route is built twice, with 8 (MX_OWN default) and with 4 entries per lane: the launch
// picks 4 for models whose contact-free island blocks take at most 192 entries (fewer registers;
// entries beyond 64 kOwn take a slower path, so larger models keep 8).
#ifndef MX_OWN
#define MX_OWN 8
#endif
constexpr int kOwn = MX_OWN;
constexpr int kSweepWords = 3 * kOwn + 4;

Layout make_layout(const MxModel& m) {
  Layout L{};
  Image I = image_layout(m);
  int at = 0;
  auto take = [&](int n) { int o = at; at += round_up(n > 0 ? n : 1, 4); return o; };   // 32-bit words
  auto takeR = [&](int n) { return take(n * kRealWords); };                               // n reals
  int nb = m.nbody, nv = m.nv, nj = m.njnt;
  L.img = take(I.words);
  L.qpos = takeR(m.nq); L.qvel = takeR(nv); L.ctrl = takeR(m.nu); L.warm = takeR(nv); L.applied = takeR(nv);
  L.xpos = takeR(3 * nb); L.xquat = takeR(4 * nb); L.xmat = takeR(9 * nb); L.xipos = takeR(3 * nb);
  L.ximat = takeR(9 * nb); L.xanchor = takeR(3 * nj); L.xaxis = takeR(3 * nj); L.scom = takeR(3 * nb);
  L.cinert = takeR(10 * nb); L.crb = takeR(10 * nb); L.cdof = takeR(6 * nv); L.cvel = takeR(6 * nb);
  L.cdofdot = takeR(6 * nv); L.cfrcb = takeR(6 * nb); L.cfrc = takeR(6 * nb);
  L.M = takeR(m.nM); L.Minv = takeR(m.nM + m.nMdamp); L.gj0 = takeR(m.nM + m.nMdamp); L.gj1 = takeR(m.nM + m.nMdamp);
  L.gxpos = takeR(3 * m.ngeom); L.gxmat = takeR(9 * m.ngeom); L.sxpos = takeR(3 * m.nsite); L.sxmat = takeR(9 * m.nsite);
  L.bias = takeR(nv); L.passive = takeR(nv); L.act = takeR(nv); L.smooth = takeR(nv); L.qacc_smooth = takeR(nv);
  L.qacc = takeR(nv); L.qcon = takeR(nv); L.tmp = takeR(nv); L.rhs = takeR(nv); L.actforce = takeR(m.nu);
  L.jacp = takeR(3 * MX_OSC_MAXDOF); L.jacr = takeR(3 * MX_OSC_MAXDOF); L.misc = take(16);
  L.tp0 = takeR(3 * nb); L.tq0 = takeR(4 * nb); L.tp1 = takeR(3 * nb); L.tq1 = takeR(4 * nb);
  L.anc0 = take(nb); L.anc1 = take(nb); L.jl = takeR(6 * nj);
  L.xfrc = takeR(6 * nb); L.cacc = takeR(6 * nb); L.cext = takeR(6 * nb); L.gcomp = takeR(nv); L.xq = takeR(nv);
  {
    int C = m.nconmax > 0 ? m.nconmax : 1, R = m.njmax > 0 ? m.njmax : 1, K = m.maxpairdof;
    bool rows = m.njmax > 0;
    L.cand = take(rows ? m.npair : 1); L.sv = take(32);
    L.bact = take(rows && m.has_body_active ? nb : 1);
    L.cpos = takeR(rows ? 3 * C : 1); L.cframe = takeR(rows ? 9 * C : 1); L.cdist = takeR(rows ? C : 1);
    L.cfric = takeR(rows ? 5 * C : 1); L.csolref = takeR(rows ? 2 * C : 1); L.csolimp = takeR(rows ? 5 * C : 1);
    L.cmargin = takeR(rows ? C : 1); L.cgeom = take(rows ? 2 * C : 1); L.cdim = take(rows ? C : 1);
    L.caddr = take(rows ? C : 1); L.cjidx = take(rows ? C * K : 1); L.cjval = takeR(rows ? 3 * C * K : 1);
    L.cjn = take(rows ? C : 1); L.cdot = takeR(rows ? 3 * C : 1);
    L.rid = take(rows ? R : 1); L.rD = takeR(rows ? R : 1); L.raref = takeR(rows ? R : 1); L.rjaref = takeR(rows ? R : 1);
    L.rjv = takeR(rows ? R : 1); L.rforce = takeR(rows ? R : 1); L.rstate = take(rows ? R : 1);
    L.rquad = takeR(rows && m.opt_cone == 1 ? 3 * R : 1);
    L.tisl = take(rows ? m.ntree : 1); L.toff = take(rows ? m.ntree : 1); L.disl = take(rows ? nv : 1); L.dloc = take(rows ? nv : 1);
    L.iblk = take(rows ? m.ntree + 1 : 1); L.isz = take(rows ? m.ntree : 1);
    L.idof = take(rows ? nv : 1); L.istart = take(rows ? m.ntree + 1 : 1);
    L.Ma = takeR(rows ? nv : 1); L.grad = takeR(rows ? nv : 1); L.search = takeR(rows ? nv : 1); L.Mv = takeR(rows ? nv : 1);
#ifdef MX_SLAB
    L.hmap = take(rows ? m.nM : 1); L.cjmap = take(rows ? C * K : 1); L.cqn = take(rows ? C : 1);
    L.hown = take(rows ? kSweepWords * kLanes : 1);
    L.ctrp = take(rows ? 2 * C + 1 : 1);
#else
    L.hmap = L.cjmap = L.cqn = L.hown = L.ctrp = -1;
#endif
    // The EPA polytope is live only inside collision, before the rows of this substep are built,
    // so it shares the row arrays' storage when it fits there.
    L.epa = -1;
    L.gpose = 0;
    L.meshw = 0;
    L.win = kWindowWords;
    if (rows && (m.nmesh > 0 || !m.boxbox_primitive)) {
      int it = m.epa_iterations > 0 ? m.epa_iterations : 0;
      L.epa_vc = 10 + 2 * it;
      L.epa_fc = 6 + 5 * it;
      int poly = round_up(cvx::poly_words(L.epa_vc, L.epa_fc), 4), need = poly + kEpaRequest + cvx::kManifoldWords;
#ifdef MX_SLAB
      L.epa = 0;                        // at the start of the LDS window
      L.epa_req = poly;
      L.win = need > L.win ? round_up(need, 4) : L.win;
      L.gpose = need;
#else
      // in reals: the polytope, the request block and the manifold's clip block
      L.epa = need * kRealWords <= L.tisl - L.rid ? L.rid : take(need * kRealWords);
      L.epa_req = L.epa + poly * kRealWords;
#endif
    }
  }
  L.nfloat = at;
  L.dbase = round_up(at * 4, 16);
  int dt = 0;
  auto dtake = [&](int n) { int o = dt; dt += round_up(n, 2); return o; };
  // the controller's state kept across substeps, then its per-substep temporaries [otmp, otmp_end)
  // (n = osc_ndof arm joints: the n x n mass block, 6 x n Jacobian, n-vectors)
  const int on = m.osc_ndof;
  L.goalpos = dtake(3); L.goalrot = dtake(9); L.grip = dtake(2); L.tau = dtake(on); L.action = dtake(7);
  L.gains = dtake(12); L.q0 = dtake(on);
  L.otmp = dt;
  L.m7 = dtake(on * on); L.minv = dtake(on * on); L.J = dtake(6 * on); L.mjt = dtake(6 * on); L.A = dtake(36);
  L.Ap = dtake(9); L.Ar = dtake(9); L.Lf = dtake(36); L.Lp = dtake(9); L.Lr = dtake(9);
  L.jbar = dtake(6 * on); L.N = dtake(on * on); L.q = dtake(on); L.qd = dtake(on); L.dbias = dtake(on);
  L.eepos = dtake(3); L.eerot = dtake(9); L.eevel = dtake(6);
  L.R = dtake(9); L.desired = dtake(6); L.wrench = dtake(6); L.pd = dtake(on); L.posture = dtake(on);
  L.work = dtake(3 * 72 + 8);
  L.otmp_end = dt;
#ifdef MX_SLAB
  if (L.win < 2 * (L.otmp_end - L.otmp)) L.win = 2 * (L.otmp_end - L.otmp);
  // actuation()'s exchange of actuator forces and qfrc_smooth
  if (L.win < 2 * m.nu + m.nv) L.win = round_up(2 * m.nu + m.nv, 4);
  // kinematics()'s pointer-jumping buffers and joint frames
  if (L.win < 16 * m.nbody + 6 * m.njnt) L.win = round_up(16 * m.nbody + 6 * m.njnt, 4);
  // velocity()'s copies of cvel, cdof_dot and the bodies' forces and subtree sums
  if (L.win < 18 * m.nbody + 6 * m.nv) L.win = round_up(18 * m.nbody + 6 * m.nv, 4);
  // com_pos()'s copies of the subtree coms, cinert and cdof, with crb_mass()'s crb
  if (L.win < 23 * m.nbody + 6 * m.nv) L.win = round_up(23 * m.nbody + 6 * m.nv, 4);
  // the contact Jacobians' inputs (make_rows(): cdof, qvel, subtree coms, dof chains)
  {
    const int need_rows = 7 * m.nv + 3 * m.nbody + (m.maxchain + 1) * m.nbody;
    if (m.njmax > 0 && L.win < need_rows) L.win = round_up(need_rows, 4);
  }
  // the islands' tables (islands(): 7 ntree + 2 words, two per contact and two per dof)
  if (m.njmax > 0 && L.win < 7 * m.ntree + 2 + 2 * m.nconmax + 2 * m.nv)
    L.win = round_up(7 * m.ntree + 2 + 2 * m.nconmax + 2 * m.nv, 4);
  // the geoms' collision records after the EPA block
  if (m.njmax > 0 && L.win < L.gpose + GP_WORDS * m.ngeom) L.win = round_up(L.gpose + GP_WORDS * m.ngeom, 4);
  // then the hull vertices (4 words each), read by every support-point search of the stage
  L.meshw = round_up(L.gpose + GP_WORDS * m.ngeom, 4);
  if (m.njmax > 0 && m.nmeshvert > 0 && L.win < L.meshw + 4 * m.nmeshvert) L.win = round_up(L.meshw + 4 * m.nmeshvert, 4);
  // row-group EPA: four (else two) blocks of a small polytope, its request / result words and a
  // box-manifold clip block, side by side at the start of the window, when they and the collision
  // records after them fit the window as sized above (the blocks never grow the window)
  L.epa_ng = 0;
  if (m.njmax > 0 && L.epa == 0) {
    L.epa_svc = kSmallPolyVerts < L.epa_vc ? kSmallPolyVerts : L.epa_vc;
    L.epa_sfc = kSmallPolyFaces < L.epa_fc ? kSmallPolyFaces : L.epa_fc;
    L.epa_gw = round_up(cvx::poly_words(L.epa_svc, L.epa_sfc), 4) + kEpaRequest + cvx::kManifoldWords;
    for (int ng = 4; ng >= 2; ng /= 2) {
      const int region = L.gpose > ng * L.epa_gw ? L.gpose : ng * L.epa_gw, meshw = round_up(region + GP_WORDS * m.ngeom, 4);
      if (meshw + 4 * m.nmeshvert <= L.win) { L.epa_ng = ng; L.gpose = region; L.meshw = meshw; break; }
    }
  }
  // contact staging (collide()): a pair table of kStagePair words per lane and kStageContact words
  // per contact of a candidate batch, over the EPA region, which is dead once the batch's EPA ends
  L.stage = -1;
  if (m.njmax > 0 && L.epa == 0 && kStagePair * kLanes + kStageContact * m.nconmax <= L.gpose) L.stage = 0;
#endif
  // Newton Hessian island blocks (packed lower triangles) and the sweep's pivot column, in FP64:
  // the blocks couple stiff contact rows with the small inertias of light objects
  {
    bool rows = m.njmax > 0;
    L.H = dtake(rows ? nv * (nv + 1) / 2 : 1);
    L.colk = dtake(rows ? nv : 1);
#ifdef MX_SLAB
    L.cq = dtake(rows ? 9 * (m.nconmax > 0 ? m.nconmax : 1) : 1);
#else
    L.cq = -1;
#endif
  }
  L.ndouble = dt;
  L.bytes = L.dbase + dt * 8;
  return L;
}

// Scalars shared by the lanes of a world (the `misc` LDS slot, 16 ints): kRank0, kGjFail and
// kFastFail head three slots each.
enum Misc { kMaxTree = 0, kCtrlErr = 1, kPinvFail = 2, kRank0 = 3, kXfrc = 6, kGjFail = 8, kFastFail = 12 };

// The launch's parameters, the kernels' one explicit argument.  Every function reads them in place
// in the kernel argument segment (scalar loads from constant memory), so the functions the kernel
// calls, inlined or not, need no private copy of them and the world context below holds no data.
struct Params {
  MxModel m;
  MxData d;
  Layout L;
  Image I;
  int substeps, flags;
  const int32_t* mask;
  MxObsPlan obs;    // observation plan sampled after every substep (nspec 0: none)
  int pace;         // workspace route: every world resident at once, so the worlds are paced
};
typedef const __attribute__((address_space(4))) Params KParams;
typedef const __attribute__((address_space(4))) MxData KData;
typedef const __attribute__((address_space(4))) Layout KLayout;
typedef const __attribute__((address_space(4))) Image KImage;
// The explicit argument sits at offset 0 of the kernel argument segment and the hidden arguments
// follow it at the next 8-byte boundary.  The implicit-argument pointer (the hidden arguments'
// base) is passed to every function a kernel calls, whereas the segment pointer itself is only
// valid in the kernel's own body, so the block is addressed back from the former.
static_assert(sizeof(Params) % 8 == 0, "the hidden arguments must start right after the parameter block");
static_assert(sizeof(Params) <= 4096 - 256, "the parameter block and the hidden arguments fit the kernel argument segment");
__device__ __forceinline__ KParams& params() {
  typedef const __attribute__((address_space(4))) unsigned char KByte;
  return *(KParams*)((KByte*)__builtin_amdgcn_implicitarg_ptr() - sizeof(Params));
}

// The launch's dynamic LDS: the whole working set (LDS route) or the world's window (workspace route).
extern __shared__ __align__(16) unsigned char mx_lds[];

// One world's view of the launch: the world is the workgroup, every address derives from the
// parameters and the workgroup id.
struct Ctx {
  __device__ KModel& m() const { return params().m; }
  __device__ KData& d() const { return params().d; }
  __device__ KLayout& L() const { return params().L; }
  __device__ KImage& I() const { return params().I; }
  __device__ int w() const { return (int)blockIdx.x; }
  // lane of the wave: the workspace route's workgroups are one wave; the LDS route's smooth kernel
  // runs two (a mask the workspace route's stage functions, compiled out of line, would carry).
  // The workspace route recomputes it at every use, out of the optimizer's sight: per-lane
  // addresses derived from threadIdx.x are invariant across the substep loop, and hoisted out of it
  // they hold registers for the whole launch and push the stages' own values to scratch (the
  // C3 build's scratch frame went from 1280 to 976 bytes per lane, its kernel time down 6.8 %).
#ifdef MX_SLAB
  __device__ int lane() const {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
  }
#else
  __device__ int lane() const { return (int)threadIdx.x & (kLanes - 1); }
#endif
#ifdef MX_SLAB
  // this world's slab of the workspace (slab 0 holds the launch's model image; the stride is a
  // multiple of 256 bytes)
  __device__ unsigned char* base() const {
    return reinterpret_cast<unsigned char*>(params().d.workspace + (size_t)(w() + 1) * params().d.workspace_doubles);
  }
  __device__ sdouble* hwin() const { return (sdouble*)mx_lds; }   // the world's LDS window
  // the world's scalar slots (misc: 16 words, sv: 32 words) in LDS after the window
  __device__ int* MISC() const { return (int*)((sint*)mx_lds + L().win); }
  __device__ int* SV() const { return (int*)((sint*)mx_lds + L().win + 16); }
  __device__ lfloat* fi() const { return (lfloat*)params().d.workspace + L().img; }   // shared by all worlds
  __device__ double* od() const { return (double*)hwin(); }
  // geom g during collision: its record in the LDS window
  __device__ const sfloat* grec(int g) const { return (const sfloat*)mx_lds + L().gpose + GP_WORDS * g; }
  __device__ const sfloat* gpos(int g) const { return grec(g) + GP_POS; }
  __device__ const sfloat* gmat(int g) const { return grec(g) + GP_MAT; }
  __device__ const sfloat* gsize(int g) const { return grec(g) + GP_SIZE; }
  __device__ int gtype(int g) const { return ((const sint*)grec(g))[GP_TYPE]; }
  __device__ float gmargin(int g) const { return grec(g)[GP_MARGIN]; }
  __device__ float ggap(int g) const { return grec(g)[GP_GAP]; }
  __device__ float grbound(int g) const { return grec(g)[GP_RBOUND]; }
  __device__ const sfloat* gvert(int g) const { return (const sfloat*)mx_lds + L().meshw + ((const sint*)grec(g))[GP_VERT]; }
  __device__ int gnvert(int g) const { return ((const sint*)grec(g))[GP_NVERT]; }
#else
  __device__ unsigned char* base() const { return mx_lds; }
  __device__ sdouble* hwin() const { return nullptr; }
  __device__ int* MISC() const { return N(L().misc); }
  __device__ int* SV() const { return N(L().sv); }
  __device__ lfloat* fi() const { return f() + L().img; }
  __device__ double* od() const { return (double*)(g() + L().otmp); }
  __device__ const sreal* gpos(int g) const { return (const sreal*)(f() + L().gxpos) + 3 * g; }
  __device__ const sreal* gmat(int g) const { return (const sreal*)(f() + L().gxmat) + 9 * g; }
  __device__ const sfloat* gsize(int g) const { return fi() + I().geom + GR * g + G_SIZE; }
  __device__ int gtype(int g) const { return gi(g, G_TYPE); }
  __device__ float gmargin(int g) const { return *gf(g, G_MARGIN); }
  __device__ float ggap(int g) const { return *gf(g, G_GAP); }
  __device__ float grbound(int g) const { return *gf(g, G_RBOUND); }
  __device__ const sfloat* gvert(int g) const {
    return fi() + I().mesh + 4 * ni()[I().meshrec + 2 * gi(g, G_DATAID)];
  }
  __device__ int gnvert(int g) const { return ni()[I().meshrec + 2 * gi(g, G_DATAID) + 1]; }
#endif
  __device__ lfloat* f() const { return (lfloat*)base(); }      // working-set floats
  __device__ lint* n() const { return (lint*)base(); }          // same storage viewed as ints
  __device__ ldouble* g() const { return (ldouble*)(base() + L().dbase); }   // working-set doubles
  __device__ lint* ni() const { return (lint*)fi(); }           // the model image (its own base)
  __device__ real* F(int off) const { return (real*)(f() + off); }   // a real array at word offset off
  __device__ lreal* R(int off) const { return (lreal*)(f() + off); }  // the same, in the working set's address space
  __device__ int* N(int off) const { return (int*)(n() + off); }
  __device__ double* D(int off) const { return (double*)(g() + off); }
  // the controller's per-substep temporaries (the LDS window on the workspace route)
  __device__ double* O(int off) const { return od() + (off - L().otmp); }
  // model image accessors (offsets within the image)
  __device__ const float* IF(int off) const { return (const float*)(fi() + off); }
  __device__ const int* IN(int off) const { return (const int*)(ni() + off); }
  __device__ int bi(int b, int k) const { return ni()[I().body + BR * b + k]; }
  __device__ const float* bf(int b, int k) const { return (const float*)(fi() + I().body + BR * b + k); }
  __device__ int ji(int j, int k) const { return ni()[I().jnt + JR * j + k]; }
  __device__ const float* jf(int j, int k) const { return (const float*)(fi() + I().jnt + JR * j + k); }
  __device__ int di(int v, int k) const { return ni()[I().dof + DR * v + k]; }
  __device__ real df(int v, int k) const { return fi()[I().dof + DR * v + k]; }
  __device__ int gi(int g_, int k) const { return ni()[I().geom + GR * g_ + k]; }
  __device__ const float* gf(int g_, int k) const { return (const float*)(fi() + I().geom + GR * g_ + k); }
  __device__ int si(int s, int k) const { return ni()[I().site + SR * s + k]; }
  __device__ const float* sf(int s, int k) const { return (const float*)(fi() + I().site + SR * s + k); }
  __device__ int ai(int a, int k) const { return ni()[I().act + AR * a + k]; }
  __device__ real af(int a, int k) const { return fi()[I().act + AR * a + k]; }
  __device__ int ti(int t, int k) const { return ni()[I().tree + TR * t + k]; }
  __device__ const int* chain(int b) const { return (const int*)(ni() + I().chain + I().chainw * b); }
  __device__ int osc_qpos(int i) const { return ni()[I().osc + i]; }
  __device__ int osc_dof(int i) const { return ni()[I().osc + MX_OSC_MAXDOF + i]; }
  __device__ int osc_act(int i) const { return ni()[I().osc + 2 * MX_OSC_MAXDOF + i]; }
  __device__ real ctrlrange(int a, int k) const { return af(a, A_CTRLRANGE + k); }
};

#ifdef MX_SLAB
__device__ __forceinline__ void sync() { __syncthreads(); }
#else
// The LDS route's stage code synchronizes its own wavefront: its workgroups hold one wave, or two
// whose waves run different stages at once (control_step_kernel_smooth) and meet at that kernel's
// own workgroup barriers only.  A wave's LDS and memory operations complete in order, so a wave
// barrier between fences that keep the compiler from moving accesses across it orders its lanes'
// accesses.
__device__ __forceinline__ void sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
#endif

// ---------------------------------------------------------------- position stage
// Forward kinematics: MuJoCo mj_kinematics semantics (reference fused leaf
// gpu/cuda/fp32/fused_kinematic_mass.cu:110-447).  Each lane first forms its body's transform
// relative to the parent (body offset, then its joints: free, slide, hinge about the anchor), then
// the tree is composed by pointer jumping: T_b <- T_anc(b) o T_b, anc(b) <- anc(anc(b)), which
// needs ceil(log2(depth)) rounds instead of one round per tree level.
__device__ void kinematics(const Ctx& c) {
  KModel& m = c.m();
  const real* qpos = c.F(c.L().qpos);
#ifdef MX_SLAB
  // Workspace route: the pointer-jumping buffers and the joints' local frames live in the LDS
  // window (free at a substep's start; 16 nbody + 6 njnt words, which the layout guarantees), so
  // each jumping round reads its ancestors' frames at LDS latency instead of the working set's.
  const int nbw = m.nbody;
  real* tp = (real*)(sfloat*)c.hwin();
  real *tq = tp + 3 * nbw, *tp1 = tq + 4 * nbw, *tq1 = tp1 + 3 * nbw;
  int* anc = (int*)(tq1 + 4 * nbw);
  int* anc1 = anc + nbw;
  real* jl = (real*)(anc1 + nbw);
#else
  real *tp = c.F(c.L().tp0), *tq = c.F(c.L().tq0), *tp1 = c.F(c.L().tp1), *tq1 = c.F(c.L().tq1);
  int *anc = c.N(c.L().anc0), *anc1 = c.N(c.L().anc1);
  real* jl = c.F(c.L().jl);
#endif
  for (int b = c.lane(); b < m.nbody; b += kLanes) {
    real pos[3] = {0.f, 0.f, 0.f}, quat[4] = {1.f, 0.f, 0.f, 0.f};
    if (b > 0) {
      const float* bp = c.bf(b, B_POS);
      const float* bq = c.bf(b, B_QUAT);
      for (int i = 0; i < 3; ++i) pos[i] = bp[i];
      for (int i = 0; i < 4; ++i) quat[i] = bq[i];
      int j0 = c.bi(b, B_JNTADR), nj = c.bi(b, B_JNTNUM);
      for (int j = j0; j < j0 + nj; ++j) {
        int qa = c.ji(j, J_QPOS), type = c.ji(j, J_TYPE);
        real* la = jl + 6 * j;
        if (type == 0) {
          for (int i = 0; i < 3; ++i) pos[i] = qpos[qa + i];
          for (int i = 0; i < 4; ++i) quat[i] = qpos[qa + 3 + i];
          normalize4(quat);
          for (int i = 0; i < 3; ++i) la[i] = pos[i];
          la[3] = 0.f; la[4] = 0.f; la[5] = 1.f;
          continue;
        }
        const float* jp = c.jf(j, J_POS);
        const float* ja = c.jf(j, J_AXIS);
        real R[9], an[3], axis[3];
        quat2mat(quat, R);
        mulmv3(R, jp, an);
        for (int i = 0; i < 3; ++i) an[i] += pos[i];
        mulmv3(R, ja, axis);
        for (int i = 0; i < 3; ++i) { la[i] = an[i]; la[3 + i] = axis[i]; }
        real delta = qpos[qa] - *c.jf(j, J_QPOS0);
        if (type == 2) {
          for (int i = 0; i < 3; ++i) pos[i] += axis[i] * delta;
        } else if (type == 3) {
          real s, co;
          r_sincos(0.5f * delta, &s, &co);
          real ql[4] = {co, ja[0] * s, ja[1] * s, ja[2] * s};
          real nq[4];
          qmul(quat, ql, nq);
          for (int i = 0; i < 4; ++i) quat[i] = nq[i];
          quat2mat(quat, R);
          real r[3];
          mulmv3(R, jp, r);
          for (int i = 0; i < 3; ++i) pos[i] = an[i] - r[i];
        }
      }
    }
    for (int i = 0; i < 3; ++i) tp[3 * b + i] = pos[i];
    for (int i = 0; i < 4; ++i) tq[4 * b + i] = quat[i];
    anc[b] = b > 0 ? c.bi(b, B_PARENT) : 0;
  }
  sync();
  int rounds = 0;
  while ((1 << rounds) < m.nlevel) ++rounds;
  for (int r = 0; r < rounds; ++r) {
    for (int b = c.lane(); b < m.nbody; b += kLanes) {
      int a = anc[b];
      real p[3], q[4];
      for (int i = 0; i < 3; ++i) p[i] = tp[3 * b + i];
      for (int i = 0; i < 4; ++i) q[i] = tq[4 * b + i];
      if (a > 0) {
        real qa[4], R[9], off[3], nq[4];
        for (int i = 0; i < 4; ++i) qa[i] = tq[4 * a + i];
        quat2mat(qa, R);
        mulmv3(R, p, off);
        for (int i = 0; i < 3; ++i) p[i] = tp[3 * a + i] + off[i];
        qmul(qa, q, nq);
        normalize4(nq);
        for (int i = 0; i < 4; ++i) q[i] = nq[i];
        a = anc[a];
      }
      for (int i = 0; i < 3; ++i) tp1[3 * b + i] = p[i];
      for (int i = 0; i < 4; ++i) tq1[4 * b + i] = q[i];
      anc1[b] = a;
    }
    sync();
    real* t;
    t = tp; tp = tp1; tp1 = t;
    t = tq; tq = tq1; tq1 = t;
    int* ta = anc; anc = anc1; anc1 = ta;
  }
  // Each loop loads its lane's inputs before it stores anything: a store to a working-set array
  // may alias any later load of the same type as far as the compiler knows, so loads left after
  // stores would each wait for a round trip to the working set.
  real *xpos = c.F(c.L().xpos), *xquat = c.F(c.L().xquat), *xmat = c.F(c.L().xmat);
  for (int b = c.lane(); b < m.nbody; b += kLanes) {
    real q[4] = {tq[4 * b], tq[4 * b + 1], tq[4 * b + 2], tq[4 * b + 3]};
    real p3[3] = {tp[3 * b], tp[3 * b + 1], tp[3 * b + 2]};
    real ip[3], iq[4];
    for (int i = 0; i < 3; ++i) ip[i] = c.bf(b, B_IPOS)[i];
    for (int i = 0; i < 4; ++i) iq[i] = c.bf(b, B_IQUAT)[i];
    normalize4(q);
    real X[9], off[3], R[9], XI[9];
    quat2mat(q, X);
    mulmv3(X, ip, off);
    quat2mat(iq, R);
    mulmm3(X, R, XI);
    for (int i = 0; i < 3; ++i) xpos[3 * b + i] = p3[i];
    for (int i = 0; i < 4; ++i) xquat[4 * b + i] = q[i];
    for (int k = 0; k < 9; ++k) xmat[9 * b + k] = X[k];
    for (int i = 0; i < 3; ++i) c.F(c.L().xipos)[3 * b + i] = p3[i] + off[i];
    for (int k = 0; k < 9; ++k) c.F(c.L().ximat)[9 * b + k] = XI[k];
  }
  sync();
  // joint anchors/axes in world, geom and site frames
  for (int j = c.lane(); j < m.njnt; j += kLanes) {
    real la[6];
    for (int i = 0; i < 6; ++i) la[i] = jl[6 * j + i];
    real* anc_w = c.F(c.L().xanchor) + 3 * j;
    real* ax_w = c.F(c.L().xaxis) + 3 * j;
    if (c.ji(j, J_TYPE) == 0) {
      for (int i = 0; i < 3; ++i) { anc_w[i] = la[i]; ax_w[i] = la[3 + i]; }
    } else {
      int p = c.bi(c.ji(j, J_BODY), B_PARENT);
      real X[9], P[3], a[3], x[3];
      for (int k = 0; k < 9; ++k) X[k] = xmat[9 * p + k];
      for (int i = 0; i < 3; ++i) P[i] = xpos[3 * p + i];
      mulmv3(X, la, a);
      mulmv3(X, la + 3, x);
      for (int i = 0; i < 3; ++i) { anc_w[i] = P[i] + a[i]; ax_w[i] = x[i]; }
    }
  }
  // a frame (pos, quat) of the model attached to body b: world position and rotation
  auto attached = [&](int b, const float* fpos, const float* fquat, real* out_pos, real* out_mat) {
    real X[9], P[3], lp[3], lq[4];
    for (int k = 0; k < 9; ++k) X[k] = xmat[9 * b + k];
    for (int i = 0; i < 3; ++i) P[i] = xpos[3 * b + i];
    for (int i = 0; i < 3; ++i) lp[i] = fpos[i];
    for (int i = 0; i < 4; ++i) lq[i] = fquat[i];
    real off[3], R[9], W[9];
    mulmv3(X, lp, off);
    quat2mat(lq, R);
    mulmm3(X, R, W);
    for (int i = 0; i < 3; ++i) out_pos[i] = P[i] + off[i];
    for (int k = 0; k < 9; ++k) out_mat[k] = W[k];
  };
  for (int gg = c.lane(); gg < m.ngeom; gg += kLanes)
    attached(c.gi(gg, G_BODY), c.gf(gg, G_POS), c.gf(gg, G_QUAT), c.F(c.L().gxpos) + 3 * gg, c.F(c.L().gxmat) + 9 * gg);
  for (int s = c.lane(); s < m.nsite; s += kLanes)
    attached(c.si(s, S_BODY), c.sf(s, S_POS), c.sf(s, S_QUAT), c.F(c.L().sxpos) + 3 * s, c.F(c.L().sxmat) + 9 * s);
  sync();
}

// Subtree com (contiguous DFS subtree sums), cinert and cdof: MuJoCo mj_comPos; reference
// gpu/cuda/dynamics/mjwarp_com_pos.cu:95 and fused_kinematic_mass.cu (centered frames).
// Loops over a body's subtree or dof chain below read kBatch entries per round (their loads issue
// together) and accumulate them in the original order, so the sums are those of the plain loop.
constexpr int kBatch = 8;

// dst[t] = src[t] for t < n, the wave's lanes striding by 64, kBatch loads in flight per lane
template <class D, class S>
__device__ __forceinline__ void wave_copy(D* dst, const S* src, int n, int lane) {
  using T = decltype(+*src);   // the element type without its address space
  for (int t0 = lane; t0 < n; t0 += kBatch * kLanes) {
    T v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) v[u] = src[t0 + u * kLanes < n ? t0 + u * kLanes : t0];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (t0 + u * kLanes < n) dst[t0 + u * kLanes] = v[u];
  }
}

// Two (or four) copies as one: every array's kBatch loads of a round issue before its stores, so the
// copies' load latencies overlap instead of following one another.
template <class D1, class S1, class D2, class S2>
__device__ __forceinline__ void wave_copy2(D1* d1, const S1* s1, int n1, D2* d2, const S2* s2, int n2, int lane) {
  using T1 = decltype(+*s1);
  using T2 = decltype(+*s2);
  const int n = n1 > n2 ? n1 : n2;
  for (int t0 = lane; t0 < n; t0 += kBatch * kLanes) {
    T1 a[kBatch];
    T2 b[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + u * kLanes;
      a[u] = t < n1 ? s1[t] : T1();
      b[u] = t < n2 ? s2[t] : T2();
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + u * kLanes;
      if (t < n1) d1[t] = a[u];
      if (t < n2) d2[t] = b[u];
    }
  }
}

// sum of a[stride * q] over q in [b, e), ascending
__device__ __forceinline__ real range_sum(const real* a, int stride, int b, int e) {
  real s = 0.f;
  for (int q0 = b; q0 < e; q0 += kBatch) {
    real x[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) x[u] = a[stride * (q0 + u < e ? q0 + u : q0)];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (q0 + u < e) s += x[u];
  }
  return s;
}

// v += sum over the chain's dofs dd (in chain order) of a[6 dd .. 6 dd + 5] * w[dd]
__device__ __forceinline__ void chain_axpy(const int* ch, const real* a, const real* w, real* v) {
  const int n = ch[0];
  for (int q0 = 1; q0 <= n; q0 += kBatch) {
    int dd[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) dd[u] = ch[q0 + u <= n ? q0 + u : q0];
    real x[kBatch][6], y[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
#pragma unroll
      for (int k = 0; k < 6; ++k) x[u][k] = a[6 * dd[u] + k];
      y[u] = w[dd[u]];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (q0 + u <= n) {
#pragma unroll
        for (int k = 0; k < 6; ++k) v[k] += x[u][k] * y[u];
      }
  }
}

__device__ void com_pos(const Ctx& c) {
  KModel& m = c.m();
  const real* xipos = c.F(c.L().xipos);
  real* scom = c.F(c.L().scom);
#ifdef MX_SLAB
  // Workspace route: the passes below and crb_mass() read the subtree coms, cinert and cdof from
  // copies in the LDS window (23 nbody + 6 nv words with crb_mass()'s crb, which the layout
  // guarantees); the working set receives them too for the later stages.
  real* wscom = (real*)(sfloat*)c.hwin();
  real* wci = wscom + 3 * m.nbody;
  real* wcd = wci + 20 * m.nbody;
#endif
  for (int b = c.lane(); b < m.nbody; b += kLanes) {
    real s[3] = {0.f, 0.f, 0.f};
    int e = b + c.bi(b, B_SUBTREE);
    for (int k0 = b; k0 < e; k0 += kBatch) {
      real mk[kBatch], x[kBatch][3];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        int k = k0 + u < e ? k0 + u : k0;
        mk[u] = *c.bf(k, B_MASS);
#pragma unroll
        for (int i = 0; i < 3; ++i) x[u][i] = xipos[3 * k + i];
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (k0 + u < e) {
#pragma unroll
          for (int i = 0; i < 3; ++i) s[i] += mk[u] * x[u][i];
        }
    }
    real sm = *c.bf(b, B_SMASS);
    for (int i = 0; i < 3; ++i) {
      const real v = sm < 1e-15f ? xipos[3 * b + i] : s[i] / sm;
      scom[3 * b + i] = v;
#ifdef MX_SLAB
      wscom[3 * b + i] = v;
#endif
    }
  }
  sync();
#ifndef MX_SLAB
  const real* wscom = scom;
#endif
  for (int b = c.lane(); b < m.nbody; b += kLanes) {
    real* ci = c.F(c.L().cinert) + 10 * b;
#ifdef MX_SLAB
    real* wc = wci + 10 * b;
#endif
    if (b == 0) {
      for (int k = 0; k < 10; ++k) ci[k] = 0.f;
#ifdef MX_SLAB
      for (int k = 0; k < 10; ++k) wc[k] = 0.f;
#endif
      continue;
    }
    const real* R = c.F(c.L().ximat) + 9 * b;
    const float* I = c.bf(b, B_INERTIA);
    real mass = *c.bf(b, B_MASS), dd[3];
    int r = c.bi(b, B_ROOT);
    for (int i = 0; i < 3; ++i) dd[i] = xipos[3 * b + i] - wscom[3 * r + i];
    real rot[9];
    for (int i = 0; i < 3; ++i)
      for (int j = 0; j < 3; ++j)
        rot[3 * i + j] = R[3 * i] * I[0] * R[3 * j] + R[3 * i + 1] * I[1] * R[3 * j + 1] + R[3 * i + 2] * I[2] * R[3 * j + 2];
    real cv[10];
    cv[0] = rot[0] + mass * (dd[1] * dd[1] + dd[2] * dd[2]);
    cv[1] = rot[4] + mass * (dd[0] * dd[0] + dd[2] * dd[2]);
    cv[2] = rot[8] + mass * (dd[0] * dd[0] + dd[1] * dd[1]);
    cv[3] = rot[1] - mass * dd[0] * dd[1];
    cv[4] = rot[2] - mass * dd[0] * dd[2];
    cv[5] = rot[5] - mass * dd[1] * dd[2];
    cv[6] = mass * dd[0]; cv[7] = mass * dd[1]; cv[8] = mass * dd[2]; cv[9] = mass;
    for (int k = 0; k < 10; ++k) ci[k] = cv[k];
#ifdef MX_SLAB
    for (int k = 0; k < 10; ++k) wc[k] = cv[k];
#endif
  }
  for (int j = c.lane(); j < m.njnt; j += kLanes) {
    int b = c.ji(j, J_BODY), da = c.ji(j, J_DOF), r = c.bi(b, B_ROOT);
    const real* an = c.F(c.L().xanchor) + 3 * j;
    const real* ax = c.F(c.L().xaxis) + 3 * j;
    real off[3];
    for (int i = 0; i < 3; ++i) off[i] = wscom[3 * r + i] - an[i];
    real* cd = c.F(c.L().cdof);
    auto put = [&](int dof, const real* o) {   // one dof's cdof, to the working set (and the window)
      for (int k = 0; k < 6; ++k) cd[6 * dof + k] = o[k];
#ifdef MX_SLAB
      for (int k = 0; k < 6; ++k) wcd[6 * dof + k] = o[k];
#endif
    };
    int type = c.ji(j, J_TYPE);
    if (type == 0) {
      const real* X = c.F(c.L().xmat) + 9 * b;
      for (int dd = 0; dd < 3; ++dd) {
        real o[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        o[3 + dd] = 1.f;
        put(da + dd, o);
      }
      for (int dd = 0; dd < 3; ++dd) {
        real o[6];
        real a3[3] = {X[dd], X[3 + dd], X[6 + dd]};
        o[0] = a3[0]; o[1] = a3[1]; o[2] = a3[2];
        cross3(a3, off, o + 3);
        put(da + 3 + dd, o);
      }
    } else if (type == 2) {
      const real o[6] = {0.f, 0.f, 0.f, ax[0], ax[1], ax[2]};
      put(da, o);
    } else if (type == 3) {
      real o[6];
      o[0] = ax[0]; o[1] = ax[1]; o[2] = ax[2];
      cross3(ax, off, o + 3);
      put(da, o);
    }
  }
  sync();
}

// Composite inertia (subtree sums) and the dense per-tree mass blocks from (dof, ancestor dof)
// pairs: MuJoCo mj_crb; reference fused_kinematic_mass.cu (CRB, CSR M) / mjwarp_mass_matrix.cu:54.
__device__ void crb_mass(const Ctx& c) {
  KModel& m = c.m();
  real* M = c.F(c.L().M);
#ifdef MX_SLAB
  // Workspace route: cinert and cdof from com_pos()'s window copies, crb in the window
  const real* ci = (real*)(sfloat*)c.hwin() + 3 * m.nbody;
  real* crb = (real*)(sfloat*)c.hwin() + 13 * m.nbody;
  const real* cdof = (real*)(sfloat*)c.hwin() + 23 * m.nbody;
#else
  const real* ci = c.F(c.L().cinert);
  real* crb = c.F(c.L().crb);
  const real* cdof = c.F(c.L().cdof);
#endif
  for (int t = c.lane(); t < 10 * m.nbody; t += kLanes) {
    int b = t / 10, k = t % 10;
    real s = 0.f;
    if (b > 0) s = range_sum(ci + k, 10, b, b + c.bi(b, B_SUBTREE));
    crb[t] = s;
  }
  for (int t = c.lane(); t < m.nM; t += kLanes) M[t] = 0.f;
  sync();
  const int* pairs = c.IN(c.I().mpair);
  for (int p = c.lane(); p < m.nMpair; p += kLanes) {
    int i = pairs[2 * p], j = pairs[2 * p + 1];
    real buf[6];
    mul_inert_vec(crb + 10 * c.di(i, D_BODY), cdof + 6 * i, buf);
    real v = 0.f;
    for (int k = 0; k < 6; ++k) v += cdof[6 * j + k] * buf[k];
    if (i == j) v += c.df(i, D_ARM);
    int t = c.di(i, D_TREE), n = c.ti(t, T_DOFNUM), a = c.ti(t, T_DOFADR);
    real* blk = M + c.ti(t, T_MADR);
    blk[(i - a) * n + (j - a)] = v;
    blk[(j - a) * n + (i - a)] = v;
  }
  sync();
}

// Inverse of every dense mass block at once (the factor/solve role of
// gpu/cuda/dynamics/mjwarp_mass_factor.cu:134-247 and mjwarp_mass_solve.cu:74-122): symmetric
// Gauss-Jordan, lanes over the concatenated block entries, one step per pivot.  With `damp` set the
// damped trees' blocks of M + h diag(dof_damping) (implicit Euler) are inverted in the same sweep,
// stored after the nM mass entries (the tree record's T_DAMPADR).  Result in out (block storage).
// kHeld: block entries per lane whose decode is held in registers (up to kHeld 64 entries; larger
// models decode per step)
template <int kHeld, class P>
__device__ void mass_inverse_in(const Ctx& c, const lreal* M, lreal* out, bool damp, real h, P* cur, P* nxt) {
  KModel& m = c.m();
  const int* ent = c.IN(c.I().mentry);
  const int total = m.nM + (damp ? m.nMdamp : 0);
  const bool held = total <= kHeld * kLanes;
  int code[kHeld];
#pragma unroll
  for (int q = 0; q < kHeld; ++q) {
    int e = c.lane() + kLanes * q;
    code[q] = held && e < total ? ent[2 * e] : -1;
  }
  for (int e0 = c.lane(); e0 < total; e0 += kBatch * kLanes) {   // loads of kBatch entries issue together
    int cd[kBatch], dof[kBatch];
    real v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      int e = e0 + u * kLanes < total ? e0 + u * kLanes : e0;
      cd[u] = ent[2 * e];
      dof[u] = ent[2 * e + 1];
      v[u] = M[e < m.nM ? e : 0];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      int e = e0 + u * kLanes;
      if (e >= total) continue;
      int n = (cd[u] >> 10) & 63, i = (cd[u] >> 16) & 63, j = (cd[u] >> 22) & 63;
      if (e >= m.nM) {   // a damped entry: the same entry of the tree's mass block, damping on the diagonal
        v[u] = M[c.ti(c.di(dof[u], D_TREE), T_MADR) + i * n + j];
        if (i == j) v[u] += h * c.df(dof[u], D_DAMP);
      }
      cur[e] = v[u];
    }
  }
  sync();
  const int maxn = m.maxtree;
  for (int k = 0; k < maxn; ++k) {
    if (held) {
#pragma unroll
      for (int q = 0; q < kHeld; ++q) {
        int cd = code[q];
        if (cd < 0) continue;
        int e = c.lane() + kLanes * q;
        int base = cd & 1023, n = (cd >> 10) & 63, i = (cd >> 16) & 63, j = (cd >> 22) & 63;
        real v = cur[e];
        if (k < n) {
          real piv = cur[base + k * n + k];
          real rowk = (j == k ? 1.f : cur[base + k * n + j]) / piv;
          real colk = cur[base + i * n + k];
          v = i == k ? rowk : (j == k ? 0.f : v) - colk * rowk;
        }
        nxt[e] = v;
      }
    } else {
      for (int e = c.lane(); e < total; e += kLanes) {
        int cd = ent[2 * e], base = cd & 1023, n = (cd >> 10) & 63, i = (cd >> 16) & 63, j = (cd >> 22) & 63;
        real v = cur[e];
        if (k < n) {
          real piv = cur[base + k * n + k];
          real rowk = (j == k ? 1.f : cur[base + k * n + j]) / piv;
          real colk = cur[base + i * n + k];
          v = i == k ? rowk : (j == k ? 0.f : v) - colk * rowk;
        }
        nxt[e] = v;
      }
    }
    sync();
    P* tmp = cur; cur = nxt; nxt = tmp;
  }
  for (int e = c.lane(); e < total; e += kLanes) out[e] = cur[e];
  sync();
}

// The Gauss-Jordan ping-pong buffers: in the working set, or (workspace route) in the world's LDS
// window, which is free outside the Newton solve.
// M and out: working-set arrays (typed with their address space: this function is not inlined)
__device__ void mass_inverse(const Ctx& c, const lreal* M, lreal* out, bool damp, real h) {
  // eight held entries per lane up to 512 block entries, sixteen beyond (measured: fewer registers
  // win where eight suffice)
  const int total = c.m().nM + (damp ? c.m().nMdamp : 0);
  const bool small = total <= 8 * kLanes;
#ifdef MX_SLAB
  if (2 * total <= c.L().win) {
    sfloat* w = (sfloat*)c.hwin();
    if (small) mass_inverse_in<8>(c, M, out, damp, h, w, w + total);
    else mass_inverse_in<16>(c, M, out, damp, h, w, w + total);
    return;
  }
#endif
  lreal* gj0 = (lreal*)(c.f() + c.L().gj0);
  lreal* gj1 = (lreal*)(c.f() + c.L().gj1);
  if (small) mass_inverse_in<8>(c, M, out, damp, h, gj0, gj1);
  else mass_inverse_in<16>(c, M, out, damp, h, gj0, gj1);
}

// y = Minv x per tree (lane per dof).
// Row i of a block-stored dense per-tree matrix (M or its inverse) times x, in column order; with
// `damped`, a damped tree's row of (M + h diag(damping))^-1.
__device__ __forceinline__ real block_row_dot(const Ctx& c, const real* Mb, const real* x, int i,
                                               bool damped = false) {
  int t = c.di(i, D_TREE), n = c.ti(t, T_DOFNUM), a = c.ti(t, T_DOFADR);
  const int dadr = damped ? c.ti(t, T_DAMPADR) : -1;
  const real* row = Mb + (dadr >= 0 ? dadr : c.ti(t, T_MADR)) + (i - a) * n;
  real s = 0.f;
  for (int k0 = 0; k0 < n; k0 += kBatch) {
    real r[kBatch], xv[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      int k = k0 + u < n ? k0 + u : k0;
      r[u] = row[k];
      xv[u] = x[a + k];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (k0 + u < n) s += r[u] * xv[u];
  }
  return s;
}

__device__ void mass_apply(const Ctx& c, const real* Minv, const real* x, real* y) {
  KModel& m = c.m();
  for (int i = c.lane(); i < m.nv; i += kLanes) y[i] = block_row_dot(c, Minv, x, i);
  sync();
}

// Spatial force [torque; force] about the subtree centre of mass of body b's root of a force f (and
// torque t, may be null) applied at b's centre of mass; zero for the world body.
__device__ __forceinline__ void point_wrench(const Ctx& c, int b, const real* f, const real* t, real* out) {
  if (b == 0) {
    for (int k = 0; k < 6; ++k) out[k] = 0.f;
    return;
  }
  const real* x = c.F(c.L().xipos) + 3 * b;
  const real* s = c.F(c.L().scom) + 3 * c.bi(b, B_ROOT);
  real off[3] = {x[0] - s[0], x[1] - s[1], x[2] - s[2]}, r[3];
  const real fv[3] = {f[0], f[1], f[2]};
  cross3(off, fv, r);
  for (int k = 0; k < 3; ++k) {
    out[k] = r[k] + (t ? t[k] : 0.f);
    out[3 + k] = fv[k];
  }
}

// Drag on body b (b > 0) moving through the model's medium, as a force and torque at its centre
// of mass in world coordinates (MuJoCo's inertia-box fluid model): the body is the box whose
// principal inertia it has (side k = sqrt(6 (I_i + I_j - I_k) / mass)); in the body's inertial
// frame, with v and w its velocity relative to the wind and its angular velocity, each axis k
// takes the Stokes terms -3 pi mu d v_k and -pi mu d^3 w_k (d the mean side) and the quadratic
// terms -rho/2 s_i s_j |v_k| v_k and -rho/64 s_k (s_i^4 + s_j^4) |w_k| w_k (i, j the other axes).
__device__ __forceinline__ void fluid_wrench(const Ctx& c, int b, real* fw, real* tw) {
  KModel& m = c.m();
  const real mass = *c.bf(b, B_MASS);
  if (!(mass >= 1e-15f)) return;
  const real* R = c.F(c.L().ximat) + 9 * b;
  const real* v = c.F(c.L().cvel) + 6 * b;
  const real* x = c.F(c.L().xipos) + 3 * b;
  const real* s = c.F(c.L().scom) + 3 * c.bi(b, B_ROOT);
  const float* I = c.bf(b, B_INERTIA);
  const real ang[3] = {v[0], v[1], v[2]};
  const real off[3] = {x[0] - s[0], x[1] - s[1], x[2] - s[2]};
  real wo[3];
  cross3(ang, off, wo);                       // cvel's linear part is taken at the root's centre
  const real lin[3] = {v[3] + wo[0] - m.opt_wind_x, v[4] + wo[1] - m.opt_wind_y, v[5] + wo[2] - m.opt_wind_z};
  real la[3], ll[3];
  for (int k = 0; k < 3; ++k) {
    la[k] = R[k] * ang[0] + R[3 + k] * ang[1] + R[6 + k] * ang[2];
    ll[k] = R[k] * lin[0] + R[3 + k] * lin[1] + R[6 + k] * lin[2];
  }
  const real scale = 6.f / mass;
  const real side[3] = {r_sqrt(r_max(1e-15f, I[1] + I[2] - I[0]) * scale),
                         r_sqrt(r_max(1e-15f, I[0] + I[2] - I[1]) * scale),
                         r_sqrt(r_max(1e-15f, I[0] + I[1] - I[2]) * scale)};
  const real pi = 3.14159265358979323846f;
  real lf[3] = {0.f, 0.f, 0.f}, lt[3] = {0.f, 0.f, 0.f};
  if (m.opt_viscosity > 0.f) {
    const real d = (side[0] + side[1] + side[2]) / 3.f;
    for (int k = 0; k < 3; ++k) {
      lt[k] = -la[k] * d * d * d * pi * m.opt_viscosity;
      lf[k] = -3.f * ll[k] * d * pi * m.opt_viscosity;
    }
  }
  if (m.opt_density > 0.f) {
    for (int k = 0; k < 3; ++k) {
      const int i = k == 0 ? 1 : 0, j = k == 2 ? 1 : 2;
      const real si2 = side[i] * side[i], sj2 = side[j] * side[j];
      lf[k] -= 0.5f * m.opt_density * side[i] * side[j] * r_abs(ll[k]) * ll[k];
      lt[k] -= m.opt_density * side[k] * (si2 * si2 + sj2 * sj2) * r_abs(la[k]) * la[k] / 64.f;
    }
  }
  for (int k = 0; k < 3; ++k) {
    fw[k] = R[3 * k] * lf[0] + R[3 * k + 1] * lf[1] + R[3 * k + 2] * lf[2];
    tw[k] = R[3 * k] * lt[0] + R[3 * k + 1] * lt[1] + R[3 * k + 2] * lt[2];
  }
}

// Generalized force of per-body spatial forces w (6 per body, about each root's subtree centre of
// mass): out[i] = cdof_i . (sum of w over the subtree of dof i's body), the transpose of the bodies'
// Jacobians at one pass (subtree sums in `cfrc`, free outside the bias computation).
__device__ void body_wrench_dofs(const Ctx& c, const real* w, real* out) {
  KModel& m = c.m();
  real* sum = c.F(c.L().cfrc);
  for (int t = c.lane(); t < 6 * m.nbody; t += kLanes) {
    int b = t / 6, k = t % 6;
    sum[t] = b > 0 ? range_sum(w + k, 6, b, b + c.bi(b, B_SUBTREE)) : 0.f;
  }
  sync();
  const real* cdof = c.F(c.L().cdof);
  for (int i = c.lane(); i < m.nv; i += kLanes) {
    const real* s6 = sum + 6 * c.di(i, D_BODY);
    real v = 0.f;
    for (int k = 0; k < 6; ++k) v += cdof[6 * i + k] * s6[k];
    out[i] = v;
  }
  sync();
}

// ---------------------------------------------------------------- velocity stage
// cvel, cdof_dot, RNE bias forces and passive forces: MuJoCo mj_comVel + mj_rne(0) + mj_passive;
// reference gpu/cuda/fp32/fused_motion_passive.cu:43-387 / fused_motion.cu:14 / mjwarp_passive.cu.
__device__ void velocity(const Ctx& c) {
  KModel& m = c.m();
  const real* qvel = c.F(c.L().qvel);
  const real* cdof = c.F(c.L().cdof);
  real* cvel = c.F(c.L().cvel);
  real* cdd = c.F(c.L().cdofdot);
#ifdef MX_SLAB
  // Workspace route: the stage's own passes read cvel, cdof_dot, the bodies' forces and their
  // subtree sums from copies in the LDS window (free between the rows and the controller; 18 nbody
  // + 6 nv words, which the layout guarantees); cvel and cdof_dot also go to the working set for
  // the post-constraint stage.
  real* wcvel = (real*)(sfloat*)c.hwin();
  real* wcdd = wcvel + 6 * m.nbody;
  real* cfb = wcdd + 6 * m.nv;
  real* cfrc = cfb + 6 * m.nbody;
#else
  real* wcvel = cvel;
  real* wcdd = cdd;
  real* cfb = c.F(c.L().cfrcb);
  real* cfrc = c.F(c.L().cfrc);
#endif
  for (int b = c.lane(); b < m.nbody; b += kLanes) {
    real v[6] = {0, 0, 0, 0, 0, 0};
    chain_axpy(c.chain(b), cdof, qvel, v);
    for (int k = 0; k < 6; ++k) cvel[6 * b + k] = v[k];
#ifdef MX_SLAB
    for (int k = 0; k < 6; ++k) wcvel[6 * b + k] = v[k];
#endif
  }
  sync();
  // cdof_dot = (velocity before this dof) x cdof: the parent's cvel plus earlier dofs of the same
  // body; the three rotations of a free joint all use the velocity after its translations.
  for (int i = c.lane(); i < m.nv; i += kLanes) {
    int b = c.di(i, D_BODY), j = c.di(i, D_JNT), da = c.ji(j, J_DOF), p = c.bi(b, B_PARENT);
    real v[6];
    for (int k = 0; k < 6; ++k) v[k] = wcvel[6 * p + k];
    int first = c.bi(b, B_DOFADR), stop = i;
    if (c.ji(j, J_TYPE) == 0) stop = i - da >= 3 ? da + 3 : i;
    for (int dd = first; dd < stop; ++dd)
      for (int k = 0; k < 6; ++k) v[k] += cdof[6 * dd + k] * qvel[dd];
    real o[6];
    cross_motion(v, cdof + 6 * i, o);
    for (int k = 0; k < 6; ++k) cdd[6 * i + k] = o[k];
#ifdef MX_SLAB
    for (int k = 0; k < 6; ++k) wcdd[6 * i + k] = o[k];
#endif
  }
  sync();
  const real* ci = c.F(c.L().cinert);
  real g[3] = {0.f, 0.f, 0.f};
  if (!(m.opt_disableflags & (1 << 6))) { g[0] = -m.opt_gravity_x; g[1] = -m.opt_gravity_y; g[2] = -m.opt_gravity_z; }
  for (int b = c.lane(); b < m.nbody; b += kLanes) {
    if (b == 0) { for (int k = 0; k < 6; ++k) cfb[k] = 0.f; continue; }
    real a[6] = {0, 0, 0, g[0], g[1], g[2]};
    chain_axpy(c.chain(b), wcdd, qvel, a);
    real f1[6], h[6], f2[6];
    mul_inert_vec(ci + 10 * b, a, f1);
    mul_inert_vec(ci + 10 * b, wcvel + 6 * b, h);
    cross_force(wcvel + 6 * b, h, f2);
    for (int k = 0; k < 6; ++k) cfb[6 * b + k] = f1[k] + f2[k];
  }
  sync();
  for (int t = c.lane(); t < 6 * m.nbody; t += kLanes) {
    int b = t / 6, k = t % 6;
    real s = 0.f;
    if (b > 0) s = range_sum(cfb + k, 6, b, b + c.bi(b, B_SUBTREE));
    cfrc[t] = s;
  }
  sync();
  const real* qpos = c.F(c.L().qpos);
  for (int i = c.lane(); i < m.nv; i += kLanes) {
    real s = 0.f;
    for (int k = 0; k < 6; ++k) s += cdof[6 * i + k] * cfrc[6 * c.di(i, D_BODY) + k];
    c.F(c.L().bias)[i] = s;
    real p = 0.f;
    if (!(m.opt_disableflags & (1 << 5))) {
      int j = c.di(i, D_JNT), type = c.ji(j, J_TYPE);
      real stiff = *c.jf(j, J_STIFF);
      if ((type == 2 || type == 3) && stiff != 0.f) p -= stiff * (qpos[c.ji(j, J_QPOS)] - *c.jf(j, J_SPRING));
      p -= c.df(i, D_DAMP) * qvel[i];
    }
    c.F(c.L().passive)[i] = p;
  }
  sync();
  // gravity compensation (MuJoCo mj_gravcomp; reference mjwarp_queries.cu:55): -gravity * mass *
  // gravcomp at each body's centre of mass, into the passive force (mjwarp_passive.cu:57) or, for
  // joints that report it as actuator force, kept for actuation() (mjwarp_actuation.cu:54)
  if (m.has_gravcomp && !(m.opt_disableflags & (1 << 6))) {
    real* w = c.F(c.L().cext);
    for (int b = c.lane(); b < m.nbody; b += kLanes) {
      const real gc = b > 0 ? m.body_gravcomp[b] * *c.bf(b, B_MASS) : 0.f;
      const real f[3] = {-m.opt_gravity_x * gc, -m.opt_gravity_y * gc, -m.opt_gravity_z * gc};
      point_wrench(c, b, f, nullptr, w + 6 * b);
    }
    sync();
    body_wrench_dofs(c, w, c.F(c.L().gcomp));
    for (int i = c.lane(); i < m.nv; i += kLanes)
      if (!m.jnt_actgravcomp[c.di(i, D_JNT)]) c.F(c.L().passive)[i] += c.F(c.L().gcomp)[i];
    sync();
  }
  // fluid forces of the inertia-box model, into the passive force (MuJoCo mj_passive; reference
  // gpu/cuda/fp32/fused_motion_passive.cu:253-330 and :350-372).  The dof projection goes through
  // `xq`, which the applied-wrench projection below overwrites before anything reads it.
  if (m.has_fluid && !(m.opt_disableflags & (1 << 5))) {
    real* w = c.F(c.L().cext);
    for (int b = c.lane(); b < m.nbody; b += kLanes) {
      real f[3] = {0.f, 0.f, 0.f}, t[3] = {0.f, 0.f, 0.f};
      if (b > 0) fluid_wrench(c, b, f, t);
      point_wrench(c, b, f, t, w + 6 * b);
    }
    sync();
    real* q = c.F(c.L().xq);
    body_wrench_dofs(c, w, q);
    for (int i = c.lane(); i < m.nv; i += kLanes) c.F(c.L().passive)[i] += q[i];
    sync();
  }
  // applied Cartesian wrenches (xfrc_applied at the bodies' centres of mass) on the dofs, added to
  // qfrc_smooth by actuation() (MuJoCo mj_xfrcAccumulate)
  if (c.MISC()[kXfrc]) {
    real* w = c.F(c.L().cext);
    const real* x = c.F(c.L().xfrc);
    for (int b = c.lane(); b < m.nbody; b += kLanes) point_wrench(c, b, x + 6 * b, x + 6 * b + 3, w + 6 * b);
    sync();
    body_wrench_dofs(c, w, c.F(c.L().xq));
  }
}

// ---------------------------------------------------------------- FP64 operational-space control
// Lane-parallel symmetric Gauss-Jordan inversion of up to three SPD operands at once (the OSC's
// M^-1, or A, A_pos, A_ori).  Lane `e` owns entry e of the concatenated problems.  Step k:
// row k <- (row k with a_kk := 1) / a_kk;  row i != k <- (row i with a_ik := 0) - a_ik * row k.
// A pivot that is not positive and finite marks the problem failed (flag in misc[kGjFail + q]).
struct GJProblem { int base, n, first; };

template <class C>
__device__ void gj_inverse(const C& c, const double* in, double* out, GJProblem p0, GJProblem p1,
                           GJProblem p2, int nprob) {
  int lane = c.lane();
  int which = -1, n = 0, base = 0, e = 0;
  if (nprob > 0 && lane >= p0.first && lane < p0.first + p0.n * p0.n) { which = 0; n = p0.n; base = p0.base; e = lane - p0.first; }
  if (nprob > 1 && lane >= p1.first && lane < p1.first + p1.n * p1.n) { which = 1; n = p1.n; base = p1.base; e = lane - p1.first; }
  if (nprob > 2 && lane >= p2.first && lane < p2.first + p2.n * p2.n) { which = 2; n = p2.n; base = p2.base; e = lane - p2.first; }
  int i = which >= 0 ? e / n : 0, j = which >= 0 ? e % n : 0;
  double a = which >= 0 ? in[base + e] : 0.0;
  int bad = 0;
  int maxn = p0.n;
  if (nprob > 1 && p1.n > maxn) maxn = p1.n;
  if (nprob > 2 && p2.n > maxn) maxn = p2.n;
  int* fail = c.MISC() + kGjFail;
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
  if (lane < 3) fail[lane] = 0;
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
// the float steps are kept unfused so that they round exactly as the CPU restatement does.  Float
// in every build, the FP64 route's included: the rounding is robosuite's.
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

// Component k (0..5) of world w's pose delta: robosuite's Controller.scale_action (the reference's
// action_component, gpu/cuda/control/osc_solver.cu:38-47).  Without ranges (osc_action_scaled = 0)
// OSC_POSE's defaults: 0.05 m and 0.5 rad per unit action clipped to [-1, 1]; with them, the clipped
// action's offset from the input range's centre times the output/input width ratio, plus the output
// range's centre, in robosuite's order of operations.
template <class M, class D>
__device__ double scaled_action(const M& m, const D& d, size_t w, int k) {
#pragma clang fp contract(off)
  const double a = d.osc_action[7 * w + k];
  if (!m.osc_action_scaled) return (k < 3 ? 0.05 : 0.5) * clip1(a);
  const double* p = d.osc_action_scale + MX_OSC_ACTION_SCALE * w;
  const double lo = p[k], hi = p[6 + k], olo = p[12 + k], ohi = p[18 + k];
  const double x = isnan(a) ? a : fmin(hi, fmax(lo, a));
  return (x - (hi + lo) * 0.5) * (fabs(ohi - olo) / fabs(hi - lo)) + (ohi + olo) * 0.5;
}

template <bool kSplit, class C>
__device__ void control_solve(const C& c, int policy, real* ctrl);
template <class C>
__device__ void control_torque(const C& c, real* ctrl);

// Controller gather (EE site Jacobian, n x n M and 6 x n J of the n = osc_ndof arm joints, q, qdot,
// bias, EE pose/velocity in FP32 as the reference's control_drive,
// gpu/cuda/fp32/fused_control_drive.cu:34-300) and the FP64 robosuite
// OSC_POSE (gpu/cuda/control/osc_solver.cu:309-678): M^-1, A = J M^-1 J^T, Lambda = pinv(A) (full,
// pos, ori), J-bar, nullspace N, goal update at the policy substep, uncoupled wrench, posture
// torque, clipping, gripper.  Writes ctrl[osc_actuator] in LDS.  kSplit: the controller without the
// bias force, which then needs only the position stage's fields; it writes the gripper's ctrl and
// leaves the arm torques' two bias-free terms to control_bias(), which adds the bias force (the
// velocity stage's) and writes the arm's ctrl.
template <bool kSplit>
__device__ void control(const Ctx& c, int policy, bool publish) {
  KModel& m = c.m();
  const int lane = c.lane();
  int* misc = c.MISC();
  const real* cdof = c.F(c.L().cdof);
  const real* scom = c.F(c.L().scom);
  const real* qvel = c.F(c.L().qvel);
  int site = m.osc_site, sb = c.si(site, S_BODY), root = c.bi(sb, B_ROOT);
  const real* sp = c.F(c.L().sxpos) + 3 * site;
  const real sp0 = sp[0], sp1 = sp[1], sp2 = sp[2];
  const real off[3] = {sp0 - scom[3 * root], sp1 - scom[3 * root + 1], sp2 - scom[3 * root + 2]};
  const int on = m.osc_ndof;   // arm joints driven by the controller (at most 8)
  const int* ch = c.chain(sb);
  const int nch = ch[0] < kLanes ? ch[0] : kLanes;   // the EE body's ancestor dofs
  // Every input is gathered by all lanes at once, so that independent loads share their latency:
  // lane l holds ancestor dof l of the EE body (its velocity term), controlled dof l (its Jacobian
  // column, position, velocity and bias) and mass entry (l / on, l % on).
  const int dd = lane < nch ? ch[1 + lane] : 0;
  const int dv = c.osc_dof(lane < on ? lane : 0), qa = c.osc_qpos(lane < on ? lane : 0);
  const int mi = lane < on * on ? lane / on : 0, mj = lane < on * on ? lane % on : 0;
  const int dvi = c.osc_dof(mi), dvj = c.osc_dof(mj);
  real ca[6], cv[6];
  for (int k = 0; k < 6; ++k) { ca[k] = cdof[6 * dd + k]; cv[k] = cdof[6 * dv + k]; }
  const real qvd = qvel[dd], qpv = c.F(c.L().qpos)[qa], qvv = qvel[dv];
  const real bv = kSplit ? 0.f : c.F(c.L().bias)[dv];
  const real rot = c.F(c.L().sxmat)[9 * site + (lane < 9 ? lane : 0)];
  const int ti = c.di(dvi, D_TREE), tj = c.di(dvj, D_TREE);
  const int n = c.ti(ti, T_DOFNUM), a = c.ti(ti, T_DOFADR), madr = c.ti(ti, T_MADR);
  const real mv = tj == ti ? c.F(c.L().M)[madr + (dvi - a) * n + (dvj - a)] : 0.f;
  // EE velocity over the ancestor dofs, summed in chain order (each lane holds one dof's terms)
  real val[6];
  {
    real t[3];
    cross3(ca, off, t);
    for (int r = 0; r < 3; ++r) { val[r] = ca[3 + r] + t[r]; val[3 + r] = ca[r]; }
  }
  real ev[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  bool anc = false;   // controlled dof `lane` is an ancestor of the EE body
  for (int q = 0; q < nch; ++q) {
    const real qq = read_lane(qvd, q);
    for (int r = 0; r < 6; ++r) ev[r] += read_lane(val[r], q) * qq;
    anc |= read_lane(dd, q) == dv;
  }
  double* gm = c.O(c.L().m7);
  double* gJ = c.O(c.L().J);
  if (lane < on) {   // EE site Jacobian column, and the arm joint's state
    real t[3];
    cross3(cv, off, t);
    for (int k = 0; k < 3; ++k) {
      gJ[k * on + lane] = anc ? cv[3 + k] + t[k] : 0.f;
      gJ[(3 + k) * on + lane] = anc ? cv[k] : 0.f;
    }
    c.O(c.L().q)[lane] = qpv; c.O(c.L().qd)[lane] = qvv;
    if (!kSplit) c.O(c.L().dbias)[lane] = bv;
  }
  if (lane < 6) {
    real e = ev[0];
    for (int r = 1; r < 6; ++r) e = lane == r ? ev[r] : e;
    c.O(c.L().eevel)[lane] = e;
  }
  if (lane < 3) c.O(c.L().eepos)[lane] = lane == 0 ? sp0 : lane == 1 ? sp1 : sp2;
  if (lane < 9) c.O(c.L().eerot)[lane] = rot;
  if (lane < on * on) gm[lane] = mv;
  sync();
  if (publish) {   // the controller inputs of the launch's last substep (FP32 values held in FP64)
    KData& d = c.d();
    const size_t w = c.w();
    if (lane < on * on) d.osc_mass[on * on * w + lane] = (float)gm[lane];
    if (lane < 6 * on) d.osc_jac[6 * on * w + lane] = (float)gJ[lane];
    if (lane < on) {
      d.osc_q[on * w + lane] = (float)c.O(c.L().q)[lane];
      d.osc_qvel[on * w + lane] = (float)c.O(c.L().qd)[lane];
      if (!kSplit) d.osc_bias[on * w + lane] = (float)c.O(c.L().dbias)[lane];
    }
    if (lane < 3) d.osc_ee_pos[3 * w + lane] = (float)c.O(c.L().eepos)[lane];
    if (lane < 9) d.osc_ee_rot[9 * w + lane] = (float)c.O(c.L().eerot)[lane];
    if (lane < 6) d.osc_ee_vel[6 * w + lane] = (float)c.O(c.L().eevel)[lane];
  }
  control_solve<kSplit>(c, policy, c.F(c.L().ctrl));
}

// The end of the split controller (control<true>) that needs the bias force: gathers qfrc_bias of the arm dofs (published
// with the other controller inputs at the launch's last substep) and forms the arm's torques and
// ctrl (control_torque()).
__device__ void control_bias(const Ctx& c, bool publish) {
  KModel& m = c.m();
  const int lane = c.lane(), on = m.osc_ndof;
  if (lane < on) {
    const real bb = c.F(c.L().bias)[c.osc_dof(lane)];
    c.O(c.L().dbias)[lane] = bb;
    if (publish) c.d().osc_bias[on * (size_t)c.w() + lane] = bb;
  }
  control_torque(c, c.F(c.L().ctrl));
}

// The FP64 OSC proper, on the controller inputs in the O() temporaries (m7, J, q, qd, dbias, eepos,
// eerot, eevel) and the state in D() (goal, gripper, action, gains, q0, tau); writes tau, ctrl and,
// at a policy substep, the goal.  C: the step kernel's world context, or the standalone controller
// kernel's (mx_osc).
template <bool kSplit, class C>
__device__ void control_solve(const C& c, int policy, real* ctrl) {
  KModel& m = c.m();
  const int lane = c.lane();
  int* misc = c.MISC();
  const double* gm = c.O(c.L().m7);
  const double* gJ = c.O(c.L().J);
  if (misc[kCtrlErr] != 0) return;
  const int on = m.osc_ndof;   // arm joints (n): M is n x n, J 6 x n
  gj_inverse(c, gm, c.O(c.L().minv), GJProblem{0, on, 0}, GJProblem{0, 0, 64}, GJProblem{0, 0, 64}, 1);
  if (misc[kGjFail]) {
    sync();
    if (lane == 0) misc[kCtrlErr] = MX_OSC_SINGULAR_MASS;
    sync();
    return;
  }
  const double* minv = c.O(c.L().minv);
  double* mjt = c.O(c.L().mjt);
  if (lane < 6 * on) {      // M^-1 J^T (n x 6)
    int i = lane / 6, col = lane % 6;
    double s = 0;
    for (int k = 0; k < on; ++k) s += minv[i * on + k] * gJ[col * on + k];
    mjt[lane] = s;
  }
  sync();
  double* A = c.O(c.L().A);
  if (lane < 36) {      // A = J M^-1 J^T
    int r = lane / 6, col = lane % 6;
    double s = 0;
    for (int k = 0; k < on; ++k) s += gJ[r * on + k] * mjt[k * 6 + col];
    A[lane] = s;
    if (r < 3 && col < 3) c.O(c.L().Ap)[r * 3 + col] = s;
    if (r >= 3 && col >= 3) c.O(c.L().Ar)[(r - 3) * 3 + col - 3] = s;
  }
  sync();
  // A, A_pos, A_ori live contiguously (A then Ap then Ar); Lf, Lp, Lr likewise.
  gj_inverse(c, c.O(c.L().A), c.O(c.L().Lf), GJProblem{0, 6, 0}, GJProblem{c.L().Ap - c.L().A, 3, 36},
             GJProblem{c.L().Ar - c.L().A, 3, 45}, 3);
  if (lane < 3) {
    const double* src = lane == 0 ? c.O(c.L().A) : (lane == 1 ? c.O(c.L().Ap) : c.O(c.L().Ar));
    const double* inv = lane == 0 ? c.O(c.L().Lf) : (lane == 1 ? c.O(c.L().Lp) : c.O(c.L().Lr));
    int n = lane == 0 ? 6 : 3;
    bool fast = !misc[kGjFail + lane];
    if (fast) {
      double ta = 0, ti = 0;
      for (int i = 0; i < n; ++i) { ta += src[i * n + i]; ti += inv[i * n + i]; }
      fast = ti > 0 && ta * ti <= 1e13;
    }
    misc[kRank0 + lane] = n;
    misc[kFastFail + lane] = fast ? 0 : 1;
  }
  sync();
  if (lane < 3 && misc[kFastFail + lane]) {
    const double* src = lane == 0 ? c.O(c.L().A) : (lane == 1 ? c.O(c.L().Ap) : c.O(c.L().Ar));
    double* inv = lane == 0 ? c.O(c.L().Lf) : (lane == 1 ? c.O(c.L().Lp) : c.O(c.L().Lr));
    int n = lane == 0 ? 6 : 3, rank = 0;
    double* work = c.O(c.L().work) + 72 * lane;
    int ok = jacobi_pinv(src, n, inv, &rank, work, work + 36);
    misc[kRank0 + lane] = rank;
    if (!ok) atomicOr(&misc[kPinvFail], 1);
  }
  sync();
  if (misc[kPinvFail]) {
    sync();
    if (lane == 0) misc[kCtrlErr] = MX_OSC_PINV_FAILED;
    sync();
    return;
  }
  const double* Lf = c.O(c.L().Lf);
  double* jbar = c.O(c.L().jbar);
  if (lane < 6 * on) {      // J-bar = M^-1 J^T Lambda (n x 6)
    int i = lane / 6, col = lane % 6;
    double s = 0;
    for (int k = 0; k < 6; ++k) s += mjt[i * 6 + k] * Lf[k * 6 + col];
    jbar[lane] = s;
  }
  // goal update (policy substep), from the scaled pose delta: goal_pos = ee + delta[0:3]; goal_rot =
  // R(delta[3:6]) ee_rot when a rotation component is nonzero (NaN included), else kept, as robosuite's
  // set_goal and the reference (gpu/cuda/control/osc_solver.cu:570-583)
  double* gp = c.D(c.L().goalpos);
  double* gr = c.D(c.L().goalrot);
  const double* eep = c.O(c.L().eepos);
  const double* eer = c.O(c.L().eerot);
  const double* action = c.D(c.L().action);
  const bool rotate = action[3] != 0.0 || action[4] != 0.0 || action[5] != 0.0;
  if (policy && lane == 48) {
    for (int k = 0; k < 3; ++k) gp[k] = eep[k] + action[k];
    if (rotate) rotation_delta(action[3], action[4], action[5], c.O(c.L().R));
  }
  sync();
  if (policy && rotate && lane < 9) {
    const double* R = c.O(c.L().R);
    int i = lane / 3, j = lane % 3;
    gr[lane] = R[3 * i] * eer[j] + R[3 * i + 1] * eer[3 + j] + R[3 * i + 2] * eer[6 + j];
  }
  double* Nn = c.O(c.L().N);
  for (int e = lane; e < on * on; e += kLanes) {      // N = I - J-bar J
    int i = e / on, j = e % on;
    double s = 0;
    for (int k = 0; k < 6; ++k) s += jbar[i * 6 + k] * gJ[k * on + j];
    Nn[e] = (i == j ? 1.0 : 0.0) - s;
  }
  sync();
  const double* gains = c.D(c.L().gains);
  const double* ev = c.O(c.L().eevel);
  double* desired = c.O(c.L().desired);
  double* pd = c.O(c.L().pd);
  if (lane < 3) {
    int r = lane, nx = (r + 1) % 3, ls = (r + 2) % 3;
    double er = 0;
    for (int cc = 0; cc < 3; ++cc) er += 0.5 * (eer[nx * 3 + cc] * gr[ls * 3 + cc] - eer[ls * 3 + cc] * gr[nx * 3 + cc]);
    double ep = gp[r] - eep[r];
    desired[r] = gains[r] * ep - gains[r + 6] * ev[r];
    desired[r + 3] = gains[r + 3] * er - gains[r + 9] * ev[r + 3];
  }
  if (lane >= 8 && lane < 8 + on) {
    int cc = lane - 8;
    pd[cc] = 10.0 * (c.D(c.L().q0)[cc] - c.O(c.L().q)[cc]) - 6.324555320336759 * c.O(c.L().qd)[cc];
  }
  sync();
  double* wrench = c.O(c.L().wrench);
  double* posture = c.O(c.L().posture);
  if (lane < 6) {
    double s = 0;
    if (m.osc_uncouple) {
      const double* lam = lane < 3 ? c.O(c.L().Lp) : c.O(c.L().Lr);
      int r = lane % 3, o = lane < 3 ? 0 : 3;
      for (int k = 0; k < 3; ++k) s += lam[r * 3 + k] * desired[o + k];
    } else {
      for (int k = 0; k < 6; ++k) s += Lf[lane * 6 + k] * desired[k];
    }
    wrench[lane] = s;
  }
  if (lane >= 8 && lane < 8 + on) {
    int r = lane - 8;
    double s = 0;
    for (int k = 0; k < on; ++k) s += gm[r * on + k] * pd[k];
    posture[r] = s;
  }
  sync();
  if (lane < on) {
    double task = 0, null = 0;
    for (int k = 0; k < 6; ++k) task += gJ[k * on + lane] * wrench[k];
    for (int k = 0; k < on; ++k) null += Nn[k * on + lane] * posture[k];
    if (kSplit) {   // the bias-free terms, for control_torque()
      double* part = c.O(c.L().work);   // free after the pseudo-inverse fallback
      part[lane] = task;
      part[MX_OSC_MAXDOF + lane] = null;
    } else {
      double t = task + c.O(c.L().dbias)[lane] + null;
      c.D(c.L().tau)[lane] = t;
      int act = c.osc_act(lane);
      double lo = c.ctrlrange(act, 0), hi = c.ctrlrange(act, 1);
      double cl = isnan(t) ? t : fmin(hi, fmax(lo, t));
      ctrl[act] = (real)cl;
    }
  } else if (lane == 8) {
    double a6 = action[6];
    double sgn = isnan(a6) ? a6 : (a6 > 0 ? 1.0 : (a6 < 0 ? -1.0 : 0.0));
    double* grip = c.D(c.L().grip);
    for (int i = 0; i < 2; ++i) {
      double v = clip1(grip[i] + (double)m.osc_gripper_speed * (i == 0 ? -1.0 : 1.0) * sgn);
      grip[i] = v;
      int act = c.osc_act(on + i);
      double lo = c.ctrlrange(act, 0), hi = c.ctrlrange(act, 1);
      ctrl[act] = (real)((hi + lo) * 0.5 + (hi - lo) * 0.5 * v);
    }
  }
  sync();
}

// The arm torques tau = task + bias + nullspace from control_solve<true>()'s terms and the bias
// force in O(dbias), clipped to the actuators' ctrl ranges (the same operations, in the same order,
// as control_solve<false>()).  Nothing when the controller is in error (then control_solve() wrote
// no terms).
template <class C>
__device__ void control_torque(const C& c, real* ctrl) {
  KModel& m = c.m();
  const int lane = c.lane(), on = m.osc_ndof;
  if (c.MISC()[kCtrlErr] != 0) return;
  if (lane < on) {
    const double* part = c.O(c.L().work);
    double t = part[lane] + c.O(c.L().dbias)[lane] + part[MX_OSC_MAXDOF + lane];
    c.D(c.L().tau)[lane] = t;
    int act = c.osc_act(lane);
    double lo = c.ctrlrange(act, 0), hi = c.ctrlrange(act, 1);
    double cl = isnan(t) ? t : fmin(hi, fmax(lo, t));
    ctrl[act] = (real)cl;
  }
  sync();
}

// ---------------------------------------------------------------- actuation, smooth acceleration
// Joint-transmission actuators and qfrc_smooth, then qacc_smooth = M^-1 qfrc_smooth: reference
// gpu/cuda/fp32/fused_actuation_solve.cu:29-210 and gpu/cuda/dynamics/mjwarp_actuation.cu.
__device__ void actuation(const Ctx& c) {
  KModel& m = c.m();
  const real* qpos = c.F(c.L().qpos);
  const real* qvel = c.F(c.L().qvel);
  const real* ctrl = c.F(c.L().ctrl);
  bool off = m.opt_disableflags & (1 << 10);
#ifdef MX_SLAB
  // Workspace route: the actuator forces and qfrc_smooth pass between lanes through the LDS window
  // (free between the controller and the Newton solve; 2 nu + nv words) instead of the working set
  // in device memory, and each lane issues the loads of its first actuator and first dof (the
  // actuator's inputs, the dof's force terms, its row of M^-1 up to kRowHeld columns) before any
  // store.  Same operations in the same order as the general form below.
  constexpr int kRowHeld = 16;
  sreal* xg = (sreal*)c.hwin();         // gear x force of each actuator
  sint* xd = (sint*)(xg + m.nu);        // the actuator's dof
  sreal* xs = xg + 2 * m.nu;            // qfrc_smooth
  const int lane = c.lane();
  const bool gcomp_on = m.has_gravcomp && !(m.opt_disableflags & (1 << 6));
  const bool xfrc = c.MISC()[kXfrc] != 0;
  auto actuator = [&](int a, real& gear, int& adof) {
    gear = c.af(a, A_GEAR);
    adof = c.ai(a, A_DOF);
    real force = 0.f;
    if (!off) {
      int qa = c.ai(a, A_QPOS);
      real cv = ctrl[a];
      if (c.ai(a, A_CTRLLIM)) cv = r_min(r_max(cv, c.af(a, A_CTRLRANGE)), c.af(a, A_CTRLRANGE + 1));
      real length = gear * qpos[qa], velocity = gear * qvel[adof];
      force = c.af(a, A_GAIN) * cv;
      if (c.ai(a, A_BIAS) == 1)
        force += c.af(a, A_BIASPRM) + c.af(a, A_BIASPRM + 1) * length + c.af(a, A_BIASPRM + 2) * velocity;
      if (c.ai(a, A_FORCELIM))
        force = r_min(r_max(force, c.af(a, A_FORCERANGE)), c.af(a, A_FORCERANGE + 1));
    }
    return force;
  };
  // a dof's force terms (passive, bias, applied, gravity compensation when its joint has it, body
  // wrenches) and its tree's row of M^-1
  struct DofIn { real pas, bia, app, gc, xq; int n, a0; const real* row; };
  auto dof_in = [&](int i) {
    DofIn d;
    d.pas = c.F(c.L().passive)[i]; d.bia = c.F(c.L().bias)[i]; d.app = c.F(c.L().applied)[i];
    d.gc = gcomp_on && m.jnt_actgravcomp[c.di(i, D_JNT)] ? c.F(c.L().gcomp)[i] : 0.f;
    d.xq = xfrc ? c.F(c.L().xq)[i] : 0.f;
    int t = c.di(i, D_TREE);
    d.n = c.ti(t, T_DOFNUM); d.a0 = c.ti(t, T_DOFADR);
    d.row = c.F(c.L().Minv) + c.ti(t, T_MADR) + (i - d.a0) * d.n;
    return d;
  };
  auto dof_smooth = [&](int i, const DofIn& d) {
    real qa = 0.f;
    if (!off)   // actuators in ascending order
      for (int a = 0; a < m.nu; ++a)
        if (xd[a] == i) qa += xg[a];
    if (gcomp_on && m.jnt_actgravcomp[c.di(i, D_JNT)]) qa += d.gc;
    c.F(c.L().act)[i] = qa;
    real sm = d.pas - d.bia + d.app + qa + d.xq;
    c.F(c.L().smooth)[i] = sm;
    xs[i] = sm;
  };
  real gear0 = 0.f, force0 = 0.f, row0[kRowHeld];
  int adof0 = -1;
  DofIn d0{};
  if (lane < m.nu) force0 = actuator(lane, gear0, adof0);
  if (lane < m.nv) {
    d0 = dof_in(lane);
#pragma unroll
    for (int k = 0; k < kRowHeld; ++k) row0[k] = d0.row[k < d0.n ? k : 0];
  }
  if (lane < m.nu) {
    xg[lane] = gear0 * force0;
    xd[lane] = adof0;
    c.F(c.L().actforce)[lane] = force0;
  }
  for (int a = lane + kLanes; a < m.nu; a += kLanes) {
    real gear;
    int adof;
    real force = actuator(a, gear, adof);
    xg[a] = gear * force;
    xd[a] = adof;
    c.F(c.L().actforce)[a] = force;
  }
  sync();
  if (lane < m.nv) dof_smooth(lane, d0);
  for (int i = lane + kLanes; i < m.nv; i += kLanes) dof_smooth(i, dof_in(i));
  sync();
  // qacc_smooth = M^-1 qfrc_smooth, per tree, columns in order
  if (lane < m.nv) {
    real s = 0.f;
#pragma unroll
    for (int k = 0; k < kRowHeld; ++k)
      if (k < d0.n) s += row0[k] * xs[d0.a0 + k];
    for (int k = kRowHeld; k < d0.n; ++k) s += d0.row[k] * xs[d0.a0 + k];
    c.F(c.L().qacc_smooth)[lane] = s;
  }
  for (int i = lane + kLanes; i < m.nv; i += kLanes) {
    DofIn d = dof_in(i);
    real s = 0.f;
    for (int k = 0; k < d.n; ++k) s += d.row[k] * xs[d.a0 + k];
    c.F(c.L().qacc_smooth)[i] = s;
  }
  sync();
  return;
#endif
  for (int a = c.lane(); a < m.nu; a += kLanes) {
    real force = 0.f;
    if (!off) {
      int qa = c.ai(a, A_QPOS), da = c.ai(a, A_DOF);
      real gear = c.af(a, A_GEAR), cv = ctrl[a];
      if (c.ai(a, A_CTRLLIM)) cv = r_min(r_max(cv, c.af(a, A_CTRLRANGE)), c.af(a, A_CTRLRANGE + 1));
      real length = gear * qpos[qa], velocity = gear * qvel[da];
      force = c.af(a, A_GAIN) * cv;
      if (c.ai(a, A_BIAS) == 1)
        force += c.af(a, A_BIASPRM) + c.af(a, A_BIASPRM + 1) * length + c.af(a, A_BIASPRM + 2) * velocity;
      if (c.ai(a, A_FORCELIM))
        force = r_min(r_max(force, c.af(a, A_FORCERANGE)), c.af(a, A_FORCERANGE + 1));
    }
    c.F(c.L().actforce)[a] = force;
  }
  sync();
  const real* actforce = c.F(c.L().actforce);
  for (int i = c.lane(); i < m.nv; i += kLanes) {
    real qa = 0.f;
    if (!off)   // actuators in ascending order; four at a time so that their loads issue together
      for (int a0 = 0; a0 < m.nu; a0 += 4) {
        int dof[4];
        real gf[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          int a = a0 + q < m.nu ? a0 + q : a0;
          dof[q] = c.ai(a, A_DOF);
          gf[q] = c.af(a, A_GEAR) * actforce[a];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (a0 + q < m.nu && dof[q] == i) qa += gf[q];
      }
    // gravity compensation reported as actuator force, applied body wrenches into qfrc_smooth
    if (m.has_gravcomp && !(m.opt_disableflags & (1 << 6)) && m.jnt_actgravcomp[c.di(i, D_JNT)])
      qa += c.F(c.L().gcomp)[i];
    c.F(c.L().act)[i] = qa;
    real xq = c.MISC()[kXfrc] ? c.F(c.L().xq)[i] : 0.f;
    c.F(c.L().smooth)[i] = c.F(c.L().passive)[i] - c.F(c.L().bias)[i] + c.F(c.L().applied)[i] + qa + xq;
  }
  sync();
  mass_apply(c, c.F(c.L().Minv), c.F(c.L().smooth), c.F(c.L().qacc_smooth));
}

// ---------------------------------------------------------------- integration
// Semi-implicit Euler with implicit joint damping: MuJoCo mj_Euler; reference
// gpu/cuda/fp32/fused_euler_step.cu:35-269 and fused_tail.cu:15-90 (advance).
__device__ void euler(const Ctx& c, bool damped) {
  KModel& m = c.m();
  const real h = m.opt_timestep;
  real* qvel = c.F(c.L().qvel);
  real* qpos = c.F(c.L().qpos);
  // the lane's first joint, read before the stores below (a store may alias the image as far as
  // the compiler knows, which would hold these loads back until it)
  int jq = 0, jd = 0, jt = -1;
  if (c.lane() < m.njnt) { jq = c.ji(c.lane(), J_QPOS); jd = c.ji(c.lane(), J_DOF); jt = c.ji(c.lane(), J_TYPE); }
  // qacc' = (M + h diag(damping))^-1 (qfrc_smooth + qfrc_constraint) on damped trees, M^-1 (...) on
  // the others, i.e. qacc on those; each lane forms the sums of its row's columns itself
  for (int i = c.lane(); i < m.nv; i += kLanes) {
    const real qa = c.F(c.L().qacc)[i], qv = qvel[i];
    real acc = qa;
    if (damped) {
      int t = c.di(i, D_TREE), n = c.ti(t, T_DOFNUM), a = c.ti(t, T_DOFADR);
      const int dadr = c.ti(t, T_DAMPADR);
      const real* row = c.F(c.L().Minv) + (dadr >= 0 ? dadr : c.ti(t, T_MADR)) + (i - a) * n;
      const real* sm = c.F(c.L().smooth) + a;
      const real* qc = c.F(c.L().qcon) + a;
      real s = 0.f;
      for (int k0 = 0; k0 < n; k0 += kBatch) {
        real r[kBatch], xv[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          int k = k0 + u < n ? k0 + u : k0;
          r[u] = row[k];
          xv[u] = sm[k] + qc[k];
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
          if (k0 + u < n) s += r[u] * xv[u];
      }
      acc = s;
    }
    c.F(c.L().warm)[i] = qa;
    qvel[i] = qv + h * acc;
  }
  sync();
  for (int j = c.lane(); j < m.njnt; j += kLanes) {
    int qa = jq, da = jd, type = jt;
    if (j >= kLanes) { qa = c.ji(j, J_QPOS); da = c.ji(j, J_DOF); type = c.ji(j, J_TYPE); }
    if (type == 0) {   // every load before the first store
      real p[3], qn[4], vl[3], v[3];
      for (int k = 0; k < 3; ++k) { p[k] = qpos[qa + k]; vl[k] = qvel[da + k]; v[k] = qvel[da + 3 + k]; }
      for (int k = 0; k < 4; ++k) qn[k] = qpos[qa + 3 + k];
      real nrm = r_sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
      real axis[3] = {1.f, 0.f, 0.f}, angle = 0.f;
      if (nrm >= 1e-15f) { for (int k = 0; k < 3; ++k) axis[k] = v[k] / nrm; angle = h * nrm; }
      real s, co;
      r_sincos(0.5f * angle, &s, &co);
      real qr[4] = {co, axis[0] * s, axis[1] * s, axis[2] * s}, out[4];
      normalize4(qn);
      qmul(qn, qr, out);
      for (int k = 0; k < 3; ++k) qpos[qa + k] = p[k] + h * vl[k];
      for (int k = 0; k < 4; ++k) qpos[qa + 3 + k] = out[k];
    } else if (type == 2 || type == 3) {
      qpos[qa] += h * qvel[da];
    }
  }
  sync();
}

// ---------------------------------------------------------------- contacts, rows, Newton
// Solver scalars (the `sv` LDS slot; ints and floats share it).
enum Sv { SV_NCON = 0, SV_NEFC = 1, SV_NF = 2, SV_NL = 3, SV_NISL = 4, SV_MAXISL = 5, SV_NITER = 6, SV_OVF = 7,
          SV_FLIP = 8, SV_FLIPOK = 16,     // 8..15: the flip summary's words (low, high halves)
          SV_STAT = 20,                    // 20..23: the launch's row, contact, iteration, iteration x row sums
          SV_ISLAND = 24 };                // workspace route: the island tables of this launch are built
enum RowKind { EFC_FRICTION = 1, EFC_LIMIT = 3, EFC_FRICTIONLESS = 5, EFC_PYRAMIDAL = 6, EFC_ELLIPTIC = 7 };
enum RowState { ST_SATISFIED = 0, ST_QUADRATIC = 1, ST_LINEAR_NEG = 2, ST_LINEAR_POS = 3, ST_CONE = 4 };

// exclusive prefix sum over the lanes, and the wave total
__device__ __forceinline__ int wave_excl_scan(int v, int lane, int& total) {
  int x = wave_incl_scan(v);
  total = __builtin_amdgcn_readlane(x, kLanes - 1);
  return x - v;
}
__device__ __forceinline__ int lanes_below(unsigned long long mask, int lane) {
  return __popcll(lane ? (mask & ((~0ull) >> (64 - lane))) : 0ull);
}

// geom state for the narrowphase from the LDS frames and the model image
__device__ GeomX geom_x(const Ctx& c, int g) {
  GeomX x;
  x.type = c.gtype(g);
  const sfloat* sz = c.gsize(g);
  const auto* gp = c.gpos(g);
  const auto* gm = c.gmat(g);
  for (int k = 0; k < 3; ++k) { x.pos[k] = gp[k]; x.size[k] = sz[k]; }
  for (int k = 0; k < 9; ++k) x.mat[k] = gm[k];
  x.vert = nullptr;
  x.nvert = 0;
  x.mesh = -1;
  if (x.type == GT_MESH) {
    x.mesh = c.gi(g, G_DATAID);
    x.vert = c.gvert(g);
    x.nvert = c.gnvert(g);
  }
  return x;
}

// Narrowphase of one primitive pair: the two geoms are built from the collision records in this
// function's registers (no pointer to the caller's copies).
__device__ __noinline__ bool lane_narrowphase(const Ctx& c, int g1, int g2, real thr, RawOut& __restrict__ o) {
  const GeomX a = geom_x(c, g1), b = geom_x(c, g2);
  return narrowphase(c.m(), a, b, thr, o);
}

// ---------------------------------------------------------------- convex pairs
// A pair goes through GJK/EPA when one geom is a hull, or both are boxes and the model keeps the
// reference's default box-box route (gpu/host/backends/cuda_fp32/physics.py:90).
__device__ __forceinline__ bool convex_pair(KModel& m, int t1, int t2) {
  return t1 != GT_PLANE && (t2 == GT_MESH || (t1 == GT_BOX && t2 == GT_BOX && !m.boxbox_primitive));
}

struct ConvexLane {        // one lane's convex candidate between GJK and EPA
  int g1, g2;
  real margin, gap;
  cvx::Phase ph;
};

__device__ cvx::CGeom convex_geom(const Ctx& c, int g, cvx::V origin, real margin) {
  cvx::CGeom x;
  x.type = c.gtype(g);
  x.pos = cvx::ld(c.gpos(g)) - origin;
  x.size = cvx::ld(c.gsize(g));
  x.rot = c.gmat(g);
  x.vert = nullptr;
  x.nvert = 0;
  if (x.type == GT_MESH) {
    x.vert = c.gvert(g);
    x.nvert = c.gnvert(g);
  }
  x.cached = -1;
  x.margin = margin;
  return x;
}

// Origin of a convex pair's translated frame: the centre of the geom with the smaller bounding
// radius.  The reference translates to geom 1's centre (mjwarp_convex_collision.cuh:43-79); a
// common translation leaves the Minkowski difference, the contacts and their depths unchanged, and
// centring it on the smaller geom keeps that geom's support points short.  Then the FP32 rounding of
// the larger geom's far-away centre (a table box as geom 1, its centre 0.3-0.8 m from the contact)
// is shared by every point of a box manifold instead of differing between them, so it cannot tilt
// the contact forces of a resting box against each other.
__device__ __forceinline__ cvx::V pair_origin(const Ctx& c, int g1, int g2) {
  return cvx::ld(c.gpos(c.grbound(g2) < c.grbound(g1) ? g2 : g1));
}

// Margin, gap and detection threshold of a geom pair.  The reference's MJWarp route
// (mjwarp_contact.cuh:71-72) adds the two geoms' margins and gaps and detects contacts below
// margin + gap; MuJoCo 2.3.7 (convex_mpr; the reference's native route,
// collision/collision_dispatch.cuh:115-116, as mj_collideGeoms) takes the larger margin and the
// larger gap and detects below the margin.  Constraint rows use margin - gap either way.
struct PairMargin {
  real margin, gap, thr;
};
__device__ __forceinline__ PairMargin pair_margin(const Ctx& c, int g1, int g2) {
  if (c.m().convex_mpr) {
    const float mg = r_max(c.gmargin(g1), c.gmargin(g2));
    return {mg, r_max(c.ggap(g1), c.ggap(g2)), mg};
  }
  return {c.gmargin(g1) + c.gmargin(g2), c.ggap(g1) + c.ggap(g2),
          c.gmargin(g1) + c.gmargin(g2) + c.ggap(g1) + c.ggap(g2)};
}

// One convex pair by MPR on its lane (MuJoCo 2.3.7 collision semantics): at most one contact, at
// the margin less the penetration depth of the shapes inflated by half the margin each, its normal replaced by a
// sphere's or capsule's surface normal at the contact point (mjc_fixNormal,
// engine_collision_convex.c.txt:169-240 in the reference's vendored originals).
__device__ __noinline__ void lane_mpr(const Ctx& c, int g1, int g2, RawOut& __restrict__ o) {
  KModel& m = c.m();
  const real thr = pair_margin(c, g1, g2).thr;
  const cvx::V origin = pair_origin(c, g1, g2);
  cvx::CGeom a = convex_geom(c, g1, origin, thr), b = convex_geom(c, g2, origin, thr);
  real depth;
  cvx::V dir, pos;
  if (!cvx::mpr::penetration(a, b, m.opt_mpr_tolerance, m.opt_mpr_iterations, depth, dir, pos)) return;
  cvx::V nrm[2] = {dir, -dir};
  bool fixed[2] = {false, false};
  const int gg[2] = {g1, g2};
  const cvx::CGeom* cg[2] = {&a, &b};
  for (int i = 0; i < 2; ++i) {
    const int t = c.gtype(gg[i]);
    if (t != GT_SPHERE && t != GT_CAPSULE) continue;
    cvx::V local = cvx::rotT(cg[i]->rot, pos - cg[i]->pos);
    if (t == GT_CAPSULE) {
      const real h = cg[i]->size[1];
      local[2] = local[2] < -h ? local[2] + h : (local[2] > h ? local[2] - h : 0.f);
    }
    const real n = r_sqrt(cvx::dot(local, local));
    local = n < 1e-15f ? cvx::mk(1.f, 0.f, 0.f) : local * (1.f / n);
    nrm[i] = cvx::rot(cg[i]->rot, local);
    fixed[i] = true;
  }
  cvx::V n = dir;
  if (fixed[0] && fixed[1]) {
    cvx::V d = nrm[0] - nrm[1];
    const real len = r_sqrt(cvx::dot(d, d));
    n = len < 1e-15f ? cvx::mk(1.f, 0.f, 0.f) : d * (1.f / len);
  } else if (fixed[0]) {
    n = nrm[0];
  } else if (fixed[1]) {
    n = -nrm[1];
  }
  const cvx::V pw = pos + origin;
  raw_push(o, pw.v, n.v, thr - depth);
}

// GJK phase of one lane's pair; contacts that need no EPA are emitted at once.  Returns true
// when the pair waits for the wave's EPA.
__device__ __noinline__ bool convex_begin(const Ctx& c, int g1, int g2, ConvexLane& __restrict__ s, RawOut& __restrict__ o) {
  s.g1 = g1;
  s.g2 = g2;
  s.margin = c.gmargin(g1) + c.gmargin(g2);
  s.gap = c.ggap(g1) + c.ggap(g2);
  const cvx::V origin = pair_origin(c, g1, g2);
  cvx::CGeom a = convex_geom(c, g1, origin, s.margin), b = convex_geom(c, g2, origin, s.margin);
  s.ph = cvx::gjk_phase(c.m().opt_ccd_tolerance, s.gap, c.m().opt_ccd_iterations, a, b);
  if (s.ph.needs_epa) return true;
  if (s.ph.distance >= s.gap) return false;
  cvx::Manifold mf;
  mf.count = 1;
  mf.one[0] = s.ph.x1;
  mf.two[0] = s.ph.x2;
  mf.dir = cvx::mk(0.f, 0.f, 0.f);
  cvx::emit(o, mf, s.ph.distance + s.margin, s.margin, s.margin + s.gap, origin);
  return false;
}

// EPA of the leader lane's pair by the whole wave; the leader emits the contacts.
__device__ __noinline__ void convex_epa(const Ctx& c, ConvexLane& __restrict__ s, RawOut& __restrict__ o, bool leader) {
  KModel& m = c.m();
#ifdef MX_SLAB
  sfloat* ebase = (sfloat*)c.hwin();
  cvx::Poly p = cvx::poly_at(ebase + c.L().epa, c.L().epa_vc, c.L().epa_fc);
  sfloat* rq = ebase + c.L().epa_req;
#else
  cvx::Poly p = cvx::poly_at((sreal*)(c.f() + c.L().epa), c.L().epa_vc, c.L().epa_fc);
  sreal* rq = (sreal*)(c.f() + c.L().epa_req);
#endif
  sint* rqi = (sint*)(rq + 33) - 33;   // the request's integers (rqi[33...]) follow its 33 reals
  if (leader) {
    // a register copy first: the request's LDS stores cannot then be ordered between the reads of
    // the lane's state (a generic pointer that may alias them)
    const cvx::Gjk r = s.ph.r;
    const real smargin = s.margin, sgap = s.gap;
    const int sg1 = s.g1, sg2 = s.g2, cached1 = s.ph.cached1, cached2 = s.ph.cached2;
    const bool enclosing = s.ph.require_enclosing;
    rq[0] = smargin; rq[1] = sgap; rq[2] = r.dist;
    cvx::st(rq + 3, r.x1); cvx::st(rq + 6, r.x2);
    for (int k = 0; k < 4; ++k) { cvx::st(rq + 9 + 3 * k, r.s1[k]); cvx::st(rq + 21 + 3 * k, r.s2[k]); }
    rqi[33] = sg1; rqi[34] = sg2; rqi[35] = r.dim;
    for (int k = 0; k < 4; ++k) { rqi[36 + k] = r.v1[k]; rqi[40 + k] = r.v2[k]; }
    rqi[44] = cached1; rqi[45] = cached2; rqi[46] = enclosing;
  }
  sync();
  const real margin = rq[0], gap = rq[1];
  const int g1 = rqi[33], g2 = rqi[34];
  const cvx::V origin = pair_origin(c, g1, g2);
  cvx::CGeom a = convex_geom(c, g1, origin, margin), b = convex_geom(c, g2, origin, margin);
  a.cached = rqi[44];
  b.cached = rqi[45];
  cvx::V x1 = cvx::ld(rq + 3), x2 = cvx::ld(rq + 6);
  real dist = rq[2];
  if (c.lane() == 0) {
    cvx::Gjk r;
    r.dist = dist; r.x1 = x1; r.x2 = x2; r.dim = rqi[35];
    for (int k = 0; k < 4; ++k) {
      r.s1[k] = cvx::ld(rq + 9 + 3 * k); r.s2[k] = cvx::ld(rq + 21 + 3 * k); r.s[k] = r.s1[k] - r.s2[k];
      r.v1[k] = rqi[36 + k]; r.v2[k] = rqi[40 + k];
    }
    bool enclosing = rqi[46] != 0;
    int status = cvx::build_polytope(p, r, a, b, enclosing);
    if (status == 0 && enclosing && !cvx::encloses_origin(p)) status = 100;
    p.sc[cvx::P_STATUS] = status;
  }
  sync();
  cvx::EpaOut e{dist, 1, x1, x2, -1, false};
  cvx::V nf = cvx::mk(0.f, 0.f, 0.f);   // the EPA face's projection of the origin (x1 - x2 in exact arithmetic)
  if (p.sc[cvx::P_STATUS] == 0) {
    bool discrete = cvx::discrete_pair(a.type, b.type) && a.margin == 0.f && b.margin == 0.f;
    e = cvx::epa_expand(p, m.opt_ccd_tolerance, m.epa_iterations, a, b, discrete, cvx::WaveGroup(c.lane()));
    if (e.face >= 0) nf = cvx::ld(p.proj + 3 * e.face);
    if (!cvx::multicontact_supported(a, b)) e.face = -1;
    if (e.horizon_overflow && c.lane() == 0) c.SV()[SV_OVF] |= MX_OVERFLOW_EPA_HORIZON;
  }
  if (leader && e.distance < gap) {
    cvx::Manifold mf = cvx::single_point(e, nf);
    if (a.type == GT_BOX && b.type == GT_BOX && e.face >= 0) {
      mf = cvx::box_multicontact(p, e.face, e.x1, e.x2, a, b, rq + kEpaRequest);
      if (mf.count < 1 || (mf.count == 1 && cvx::dot(mf.dir, mf.dir) == 0.f)) mf = cvx::single_point(e, nf);
    }
    cvx::emit(o, mf, e.distance + margin, margin, margin + gap, origin);
  }
  sync();
}

// Contact material of a geom pair (contact_material, mjwarp_contact.cuh:56-101): the priority
// winner's condim and friction, else the larger of each; solref / solimp mixed by solmix (weight 1
// or 0 for a priority winner), solref by element-wise minimum when either uses the direct format;
// friction at least 1e-5.
__device__ __forceinline__ void pair_material(const Ctx& c, int g1, int g2, int& dim, real* fr, real* solref,
                                              real* solimp) {
  int pr1 = c.gi(g1, G_PRIORITY), pr2 = c.gi(g2, G_PRIORITY);
  real mix;
  if (pr1 != pr2) {
    int g = pr1 > pr2 ? g1 : g2;
    mix = pr1 > pr2 ? 1.f : 0.f;
    dim = c.gi(g, G_CONDIM);
    for (int k = 0; k < 3; ++k) fr[k] = *c.gf(g, G_FRIC + k);
  } else {
    dim = max(c.gi(g1, G_CONDIM), c.gi(g2, G_CONDIM));
    for (int k = 0; k < 3; ++k) fr[k] = r_max(*c.gf(g1, G_FRIC + k), *c.gf(g2, G_FRIC + k));
    real s1 = *c.gf(g1, G_SOLMIX), s2 = *c.gf(g2, G_SOLMIX);
    mix = s1 + s2 != 0.f ? s1 / (s1 + s2) : 0.f;
    if (s1 < 1e-15f && s2 < 1e-15f) mix = 0.5f;
    if (s1 < 1e-15f && s2 >= 1e-15f) mix = 0.f;
    if (s1 >= 1e-15f && s2 < 1e-15f) mix = 1.f;
  }
  if (*c.gf(g1, G_SOLREF) > 0.f && *c.gf(g2, G_SOLREF) > 0.f)
    for (int k = 0; k < 2; ++k) solref[k] = mix * *c.gf(g1, G_SOLREF + k) + (1.f - mix) * *c.gf(g2, G_SOLREF + k);
  else
    for (int k = 0; k < 2; ++k) solref[k] = r_min(*c.gf(g1, G_SOLREF + k), *c.gf(g2, G_SOLREF + k));
  for (int k = 0; k < 5; ++k) solimp[k] = mix * *c.gf(g1, G_SOLIMP + k) + (1.f - mix) * *c.gf(g2, G_SOLIMP + k);
  for (int k = 0; k < 3; ++k) fr[k] = r_max(1e-5f, fr[k]);
}

// EPA of up to four pending pairs at once (workspace route, when the window holds L.epa_ng
// row-group blocks): the pair of the k-th lane of `batch` is expanded by row k of the wave (lanes
// 16k..16k+15) on a small polytope in block k of the window (the polytope, then the request words,
// which the row overwrites with its result, then a box-manifold clip block), so the single-lane
// parts (polytope build, box manifold) of the four pairs also run side by side.  Returns true on a
// batch lane whose pair outgrew the small polytope; that pair is expanded again by convex_epa.
__device__ __noinline__ bool convex_epa_rows(const Ctx& c, ConvexLane& __restrict__ s, RawOut& __restrict__ o,
                                              unsigned long long batch) {
#ifdef MX_SLAB
  KModel& m = c.m();
  const int lane = c.lane(), gw = c.L().epa_gw, ps = gw - kEpaRequest - cvx::kManifoldWords;
  sfloat* win = (sfloat*)c.hwin() + c.L().epa;
  const bool mine = ((batch >> lane) & 1ull) != 0ull;
  const int rank = __popcll(batch & ((1ull << lane) - 1ull));
  if (mine) {   // the request of this lane's pair into block `rank` (as convex_epa's leader)
    const cvx::Gjk r = s.ph.r;
    const real smargin = s.margin, sgap = s.gap;
    const int sg1 = s.g1, sg2 = s.g2, cached1 = s.ph.cached1, cached2 = s.ph.cached2;
    const bool enclosing = s.ph.require_enclosing;
    sfloat* rq = win + rank * gw + ps;
    sint* rqi = (sint*)rq;
    rq[0] = smargin; rq[1] = sgap; rq[2] = r.dist;
    cvx::st(rq + 3, r.x1); cvx::st(rq + 6, r.x2);
    for (int k = 0; k < 4; ++k) { cvx::st(rq + 9 + 3 * k, r.s1[k]); cvx::st(rq + 21 + 3 * k, r.s2[k]); }
    rqi[33] = sg1; rqi[34] = sg2; rqi[35] = r.dim;
    for (int k = 0; k < 4; ++k) { rqi[36 + k] = r.v1[k]; rqi[40 + k] = r.v2[k]; }
    rqi[44] = cached1; rqi[45] = cached2; rqi[46] = enclosing;
  }
  sync();
  const int grp = lane >> 4;
  if (grp < __popcll(batch)) {
    const cvx::RowGroup g(lane);
    sfloat* blk = win + grp * gw;
    cvx::Poly p = cvx::poly_at(blk, c.L().epa_svc, c.L().epa_sfc);
    sfloat* rq = blk + ps;
    sint* rqi = (sint*)rq;
    const real margin = rq[0], gap = rq[1];
    const int g1 = rqi[33], g2 = rqi[34];
    const cvx::V origin = pair_origin(c, g1, g2);
    cvx::CGeom a = convex_geom(c, g1, origin, margin), b = convex_geom(c, g2, origin, margin);
    a.cached = rqi[44];
    b.cached = rqi[45];
    cvx::V x1 = cvx::ld(rq + 3), x2 = cvx::ld(rq + 6);
    real dist = rq[2];
    if (g.lane == 0) {
      cvx::Gjk r;
      r.dist = dist; r.x1 = x1; r.x2 = x2; r.dim = rqi[35];
      for (int k = 0; k < 4; ++k) {
        r.s1[k] = cvx::ld(rq + 9 + 3 * k); r.s2[k] = cvx::ld(rq + 21 + 3 * k); r.s[k] = r.s1[k] - r.s2[k];
        r.v1[k] = rqi[36 + k]; r.v2[k] = rqi[40 + k];
      }
      bool enclosing = rqi[46] != 0;
      int status = cvx::build_polytope(p, r, a, b, enclosing);
      if (status == 0 && enclosing && !cvx::encloses_origin(p)) status = 100;
      p.sc[cvx::P_STATUS] = status;
    }
    g.fence();
    cvx::EpaOut e{dist, 1, x1, x2, -1, false, false};
    cvx::V nf = cvx::mk(0.f, 0.f, 0.f);   // the EPA face's projection of the origin (x1 - x2 in exact arithmetic)
    if (p.sc[cvx::P_STATUS] == 0) {
      bool discrete = cvx::discrete_pair(a.type, b.type) && a.margin == 0.f && b.margin == 0.f;
      e = cvx::epa_expand(p, m.opt_ccd_tolerance, m.epa_iterations, a, b, discrete, g);
      if (e.face >= 0 && !e.redo) nf = cvx::ld(p.proj + 3 * e.face);
      if (!cvx::multicontact_supported(a, b)) e.face = -1;
    }
    // the result over the request: 0 no contact, 1 the manifold follows, 2 expand again
    if (g.lane == 0) {
      const int status = e.redo ? 2 : (e.distance < gap ? 1 : 0);
      if (status == 1) {
        cvx::Manifold mf = cvx::single_point(e, nf);
        if (a.type == GT_BOX && b.type == GT_BOX && e.face >= 0) {
          mf = cvx::box_multicontact(p, e.face, e.x1, e.x2, a, b, rq + kEpaRequest);
          if (mf.count < 1 || (mf.count == 1 && cvx::dot(mf.dir, mf.dir) == 0.f)) mf = cvx::single_point(e, nf);
        }
        rqi[2] = mf.count;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (k >= mf.count) continue;
          cvx::st(rq + 3 + 3 * k, mf.one[k]); cvx::st(rq + 15 + 3 * k, mf.two[k]); rq[27 + k] = mf.distance[k];
        }
        cvx::st(rq + 31, mf.dir);
      }
      rq[1] = e.distance;
      rqi[0] = status;
    }
  }
  sync();
  bool redo = false;
  if (mine) {
    const sfloat* rq = win + rank * gw + ps;
    const sint* rqi = (const sint*)rq;
    const int status = rqi[0];
    redo = status == 2;
    if (status == 1) {
      cvx::Manifold mf;
      mf.count = rqi[2];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (k >= mf.count) continue;
        mf.one[k] = cvx::ld(rq + 3 + 3 * k); mf.two[k] = cvx::ld(rq + 15 + 3 * k); mf.distance[k] = rq[27 + k];
      }
      mf.dir = cvx::ld(rq + 31);
      const real distance = rq[1];
      cvx::emit(o, mf, distance + s.margin, s.margin, s.margin + s.gap, pair_origin(c, s.g1, s.g2));
    }
  }
  sync();
  return redo;
#else
  return false;
#endif
}

// Broadphase over the static pair table (bounding spheres / plane half-space), narrowphase one
// candidate per lane, deterministic compaction, contact material and frame
// (gpu/cuda/collision/mjwarp_broadphase.cu:21-117, mjwarp_contact.cuh:42-120).
__device__ void collide(const Ctx& c) {
  KModel& m = c.m();
  int* sv = c.SV();
  int* cand = c.N(c.L().cand);
  const int* pairs = c.IN(c.I().pair);
#ifdef MX_SLAB
  {   // the geoms' collision records into the LDS window for the whole stage
    sfloat* gp = (sfloat*)mx_lds + c.L().gpose;
    const real* gx = c.F(c.L().gxpos);
    const real* gm = c.F(c.L().gxmat);
    for (int g = c.lane(); g < m.ngeom; g += kLanes) {   // one lane per geom: its loads issue together
      real x[GP_TYPE];
      for (int k = 0; k < 3; ++k) x[GP_POS + k] = gx[3 * g + k];
      for (int k = 0; k < 9; ++k) x[GP_MAT + k] = gm[9 * g + k];
      for (int k = 0; k < 3; ++k) x[GP_SIZE + k] = *c.gf(g, G_SIZE + k);
      const int type = c.gi(g, G_TYPE), id = c.gi(g, G_DATAID);
      const real margin = *c.gf(g, G_MARGIN), gap = *c.gf(g, G_GAP), rbound = *c.gf(g, G_RBOUND);
      int vert = 0, nvert = 0;
      if (type == GT_MESH) {
        const int* rec = c.IN(c.I().meshrec + 2 * id);
        vert = 4 * rec[0];   // words into the vertex copy
        nvert = rec[1];
      }
      sfloat* r = gp + GP_WORDS * g;
      for (int k = 0; k < GP_TYPE; ++k) r[k] = x[k];
      ((sint*)r)[GP_TYPE] = type;
      r[GP_MARGIN] = margin;
      r[GP_GAP] = gap;
      r[GP_RBOUND] = rbound;
      ((sint*)r)[GP_VERT] = vert;
      ((sint*)r)[GP_NVERT] = nvert;
    }
    wave_copy((sfloat*)mx_lds + c.L().meshw, c.fi() + c.I().mesh, 4 * m.nmeshvert, c.lane());
    sync();
  }
#endif
  int ncand = 0;
  for (int base = 0; base < m.npair; base += kLanes) {
    int p = base + c.lane();
    bool keep = false;
    if (p < m.npair) {
      int g1 = pairs[2 * p], g2 = pairs[2 * p + 1];
      const real thr = pair_margin(c, g1, g2).thr;
      const auto* c1 = c.gpos(g1);
      const auto* c2 = c.gpos(g2);
      real d[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
      if (c.gtype(g1) == GT_PLANE) {
        const auto* gm1 = c.gmat(g1);
        real n[3] = {gm1[2], gm1[5], gm1[8]};
        keep = dot3f(n, d) <= c.grbound(g2) + thr;
      } else {
        real bound = c.grbound(g1) + c.grbound(g2) + thr;
        keep = dot3f(d, d) <= bound * bound;
      }
      // heterogeneous batches: pairs touching a parked (inactive) body are masked out
      if (m.has_body_active) {
        const int* act = c.N(c.L().bact);
        keep = keep && act[c.gi(g1, G_BODY)] != 0 && act[c.gi(g2, G_BODY)] != 0;
      }
    }
    unsigned long long mask = __ballot(keep);
    if (keep) cand[ncand + lanes_below(mask, c.lane())] = p;
    ncand += __popcll(mask);
  }
  sync();
  int ncon = 0, ovf = 0;
  const int C = m.nconmax;
  for (int base = 0; base < ncand; base += kLanes) {
    int q = base + c.lane();
    RawOut o;
    o.n = 0;
    o.tangent_mask = 0u;
    int g1 = 0, g2 = 0;
    bool pending = false;
    ConvexLane cl;
    if (q < ncand) {
      int p = cand[q];
      g1 = pairs[2 * p];
      g2 = pairs[2 * p + 1];
      if (convex_pair(m, c.gtype(g1), c.gtype(g2))) {
        if (m.convex_mpr) lane_mpr(c, g1, g2, o);
        else pending = convex_begin(c, g1, g2, cl, o);
      } else {
        lane_narrowphase(c, g1, g2, pair_margin(c, g1, g2).thr, o);
      }
    }
    // pairs that need EPA: up to four at a time, each expanded by a 16-lane row of the wave on a
    // small polytope (workspace route, when the window holds them); a pair alone, and any pair
    // that outgrew its small polytope, expanded by the whole wave on the full-size one
    unsigned long long pend = __ballot(pending);
#ifdef MX_SLAB
    if (c.L().epa_ng > 1) {
      unsigned long long again = 0ull;
      while (__popcll(pend) > 1) {
        unsigned long long batch = 0ull, rest = pend;
        for (int k = 0; k < c.L().epa_ng && rest; ++k) {
          batch |= rest & (~rest + 1ull);
          rest &= rest - 1ull;
        }
        again |= __ballot(convex_epa_rows(c, cl, o, batch));
        pend = rest;
      }
      pend |= again;
    }
#endif
    for (; pend; pend &= pend - 1) {
      int leader = __ffsll((long long)pend) - 1;
      convex_epa(c, cl, o, c.lane() == leader);
    }
    int total;
    int off = wave_excl_scan(o.n, c.lane(), total);
#ifdef MX_SLAB
    if (c.L().stage >= 0) {
      // the pairs' records and their contacts into the LDS staging (each pair lane), then one lane
      // per contact writes the contact's fields: stores of consecutive slots from consecutive lanes
      sfloat* P = (sfloat*)mx_lds + c.L().stage;
      sfloat* S = P + kStagePair * kLanes;
      if (o.n) {
        int dim;
        real fr[3], solref[2], solimp[5];
        pair_material(c, g1, g2, dim, fr, solref, solimp);
        const PairMargin pm = pair_margin(c, g1, g2);
        sfloat* pe = P + kStagePair * c.lane();
        for (int k = 0; k < 3; ++k) pe[k] = fr[k];
        pe[3] = solref[0]; pe[4] = solref[1];
        for (int k = 0; k < 5; ++k) pe[5 + k] = solimp[k];
        pe[10] = pm.margin - pm.gap;
        ((sint*)pe)[11] = g1; ((sint*)pe)[12] = g2; ((sint*)pe)[13] = dim;
        for (int k = 0; k < 3; ++k) pe[14 + k] = o.tangent[k];
        ((sint*)pe)[17] = (int)o.tangent_mask;
        for (int k = 0; k < o.n; ++k) {
          const int st = off + k;
          if (ncon + st >= C) { ovf = 1; continue; }
          sfloat* se = S + kStageContact * st;
          for (int j = 0; j < 3; ++j) { se[j] = o.pos[k][j]; se[3 + j] = o.normal[k][j]; }
          se[6] = o.dist[k];
          ((sint*)se)[7] = c.lane() | (k << 8);
        }
      }
      sync();
      const int nnew = min(total, C - ncon);
      for (int st = c.lane(); st < nnew; st += kLanes) {
        const sfloat* se = S + kStageContact * st;
        const int owner = ((const sint*)se)[7], k = owner >> 8, slot = ncon + st;
        const sfloat* pe = P + kStagePair * (owner & 255);
        real nrm[3] = {se[3], se[4], se[5]}, fr9[9];
        if ((((const sint*)pe)[17] >> k) & 1) {
          real tg[3] = {pe[14], pe[15], pe[16]};
          for (int j = 0; j < 3; ++j) { fr9[j] = nrm[j]; fr9[3 + j] = tg[j]; }
          cross3(nrm, tg, fr9 + 6);
        } else {
          make_frame(nrm, fr9);
        }
        for (int j = 0; j < 3; ++j) c.F(c.L().cpos)[3 * slot + j] = se[j];
        for (int j = 0; j < 9; ++j) c.F(c.L().cframe)[9 * slot + j] = fr9[j];
        c.F(c.L().cdist)[slot] = se[6];
        real* f5 = c.F(c.L().cfric) + 5 * slot;
        f5[0] = pe[0]; f5[1] = pe[0]; f5[2] = pe[1]; f5[3] = pe[2]; f5[4] = pe[2];
        for (int j = 0; j < 2; ++j) c.F(c.L().csolref)[2 * slot + j] = pe[3 + j];
        for (int j = 0; j < 5; ++j) c.F(c.L().csolimp)[5 * slot + j] = pe[5 + j];
        c.F(c.L().cmargin)[slot] = pe[10];
        c.N(c.L().cgeom)[2 * slot] = ((const sint*)pe)[11];
        c.N(c.L().cgeom)[2 * slot + 1] = ((const sint*)pe)[12];
        c.N(c.L().cdim)[slot] = ((const sint*)pe)[13];
      }
      sync();
    } else
#endif
    {
      if (o.n) {
        int dim;
        real fr[3], solref[2], solimp[5];
        pair_material(c, g1, g2, dim, fr, solref, solimp);
        const PairMargin pm = pair_margin(c, g1, g2);
        for (int k = 0; k < o.n; ++k) {
          int slot = ncon + off + k;
          if (slot >= C) { ovf = 1; continue; }
          for (int j = 0; j < 3; ++j) c.F(c.L().cpos)[3 * slot + j] = o.pos[k][j];
          real* fr9 = c.F(c.L().cframe) + 9 * slot;
          if (o.tangent_mask & (1u << k)) {
            for (int j = 0; j < 3; ++j) { fr9[j] = o.normal[k][j]; fr9[3 + j] = o.tangent[j]; }
            cross3(o.normal[k], o.tangent, fr9 + 6);
          } else {
            make_frame(o.normal[k], fr9);
          }
          c.F(c.L().cdist)[slot] = o.dist[k];
          real* f5 = c.F(c.L().cfric) + 5 * slot;
          f5[0] = fr[0]; f5[1] = fr[0]; f5[2] = fr[1]; f5[3] = fr[2]; f5[4] = fr[2];
          for (int j = 0; j < 2; ++j) c.F(c.L().csolref)[2 * slot + j] = solref[j];
          for (int j = 0; j < 5; ++j) c.F(c.L().csolimp)[5 * slot + j] = solimp[j];
          c.F(c.L().cmargin)[slot] = pm.margin - pm.gap;
          c.N(c.L().cgeom)[2 * slot] = g1;
          c.N(c.L().cgeom)[2 * slot + 1] = g2;
          c.N(c.L().cdim)[slot] = dim;
        }
      }
    }
    ncon = min(ncon + total, C);
  }
  ovf = __any(ovf);
  if (c.lane() == 0) {
    sv[SV_NCON] = ncon;
    if (ovf) sv[SV_OVF] |= MX_OVERFLOW_NARROWPHASE;
  }
  sync();
}

struct KBI { real k, b, imp; };

// solref/solimp -> stiffness, damping, impedance (mjwarp_constraint_build.cu:22-37, refsafe on)
__device__ KBI impedance(real timestep, const real* ref, const real* imp, real position) {
  const real minimp = 0.0001f, maximp = 0.9999f, minval = 1e-15f;
  real time = r_max(ref[0], 2.f * timestep);
  real lo = r_min(r_max(imp[0], minimp), maximp), hi = r_min(r_max(imp[1], minimp), maximp);
  real width = r_max(minval, imp[2]), mid = r_min(r_max(imp[3], minimp), maximp), power = r_max(1.f, imp[4]);
  real k = ref[0] <= 0.f ? -ref[0] / r_max(minval, hi * hi) : 1.f / r_max(minval, hi * hi * time * time * ref[1] * ref[1]);
  real b = ref[1] <= 0.f ? -ref[1] / r_max(minval, hi) : 2.f / r_max(minval, hi * time);
  real x = r_abs(position) / width, r;
  if (lo == hi || imp[2] <= minval) r = 0.5f * (lo + hi);
  else if (x <= 0.f) r = lo;
  else if (x >= 1.f) r = hi;
  else if (power == 1.f) r = lo + x * (hi - lo);
  else if (x <= mid) r = r_min(r_max(lo + (1.f / r_pow(mid, power - 1.f)) * r_pow(x, power) * (hi - lo), lo), hi);
  else r = r_min(r_max(lo + (1.f - (1.f / r_pow(1.f - mid, power - 1.f)) * r_pow(1.f - x, power)) * (hi - lo), lo), hi);
  return {k, b, r};
}

__device__ __forceinline__ void publish_row(const Ctx& c, int r, real position, real imp_position, real weight,
                                            const real* ref, const real* imp, real velocity, bool friction) {
  KBI kbi = impedance(c.m().opt_timestep, ref, imp, imp_position);
  real k = friction ? 0.f : kbi.k;
  c.F(c.L().rD)[r] = 1.f / r_max(weight * (1.f - kbi.imp) / kbi.imp, 1e-15f);
  c.F(c.L().raref)[r] = -k * kbi.imp * position - kbi.b * velocity;
}

// coefficients of a contact row on the contact's (normal, tangent1, tangent2) Jacobian rows, from
// the contacts' dims and friction coefficients (working set or an LDS copy)
template <class IP, class FP>
__device__ __forceinline__ void row_coef(KModel& m, const IP* cdim, const FP* cfric, int con, int comp, real* co) {
  // selects rather than indexed stores keep `co` in registers
  int dim = cdim[con];
  if (m.opt_cone == 1 || dim == 1) {
    co[0] = comp == 0 ? 1.f : 0.f;
    co[1] = comp == 1 ? 1.f : 0.f;
    co[2] = comp == 2 ? 1.f : 0.f;
    return;
  }
  int dir = comp / 2 + 1;
  real f = cfric[5 * con + dir - 1] * (1.f - 2.f * real(comp & 1));
  co[0] = 1.f;
  co[1] = dir == 1 ? f : 0.f;
  co[2] = dir == 2 ? f : 0.f;
}
__device__ __forceinline__ void row_coef(const Ctx& c, int con, int comp, real* co) {
  row_coef(c.m(), c.N(c.L().cdim), c.F(c.L().cfric), con, comp, co);
}

// single-dof rows: rid = -1 - (dof | kind << 12), kind 0 friction, 1 limit (+1), 2 limit (-1)
__device__ __forceinline__ int single_dof(int rid, real& sign, int& kind) {
  int code = -1 - rid;
  kind = code >> 12;
  sign = kind == 2 ? -1.f : 1.f;
  return code & 4095;
}

// Constraint rows (mjwarp_constraint_build.cu:53-199) in deterministic order: dof friction rows,
// joint limits, then contacts.  Contact rows keep a 3 x K contact-frame Jacobian per contact.
__device__ __noinline__ void make_rows(const Ctx& c) {
  KModel& m = c.m();
  int* sv = c.SV();
  const real* qpos = c.F(c.L().qpos);
  const real* qvel = c.F(c.L().qvel);
  int* rid = c.N(c.L().rid);
  const int R = m.njmax;
  int nr = 0, nf = 0, nl = 0, ovf = 0;
  // dof friction rows
  if (!(m.opt_disableflags & (1 << 2)))
    for (int base = 0; base < m.nv; base += kLanes) {
      int d = base + c.lane();
      bool on = d < m.nv && c.df(d, D_FLOSS) > 0.f;
      unsigned long long mask = __ballot(on);
      int r = nr + lanes_below(mask, c.lane());
      if (on && r < R) {
        rid[r] = -1 - d;
        real ref[2] = {c.df(d, D_SOLREF), c.df(d, D_SOLREF + 1)};
        real imp[5];
        for (int k = 0; k < 5; ++k) imp[k] = c.df(d, D_SOLIMP + k);
        publish_row(c, r, 0.f, 0.f, c.df(d, D_INVW), ref, imp, qvel[d], true);
      }
      nr += __popcll(mask);
      nf += __popcll(mask);
    }
  // joint limits
  if (!(m.opt_disableflags & (1 << 3)))
    for (int base = 0; base < m.njnt; base += kLanes) {
      int j = base + c.lane();
      bool on = false;
      real position = 0.f, sign = 1.f;
      if (j < m.njnt && c.ji(j, J_LIMITED) && (c.ji(j, J_TYPE) == 2 || c.ji(j, J_TYPE) == 3)) {
        real q = qpos[c.ji(j, J_QPOS)];
        real lower = q - *c.jf(j, J_RANGE), upper = *c.jf(j, J_RANGE + 1) - q;
        position = r_min(lower, upper) - *c.jf(j, J_MARGIN);
        sign = lower < upper ? 1.f : -1.f;
        on = position < 0.f;
      }
      unsigned long long mask = __ballot(on);
      int r = nr + lanes_below(mask, c.lane());
      if (on && r < R) {
        int d = c.ji(j, J_DOF);
        rid[r] = -1 - (d | ((sign > 0.f ? 1 : 2) << 12));
        real ref[2] = {*c.jf(j, J_SOLREF), *c.jf(j, J_SOLREF + 1)};
        real imp[5];
        for (int k = 0; k < 5; ++k) imp[k] = *c.jf(j, J_SOLIMP + k);
        publish_row(c, r, position, position, c.df(d, D_INVW), ref, imp, sign * qvel[d], false);
      }
      nr += __popcll(mask);
      nl += __popcll(mask);
    }
  if (nr > R) { ovf = 1; nr = R; }
  // contacts: row addresses by an exclusive scan of the per-contact row counts
  const int ncon = sv[SV_NCON], K = m.maxpairdof;
  const real ratio2 = 1.f / m.opt_impratio;
#ifdef MX_SLAB
  // the contact Jacobians' inputs in the LDS window (free between collision and the controller):
  // cdof, qvel, subtree coms and the bodies' dof chains
  const int chainw = c.I().chainw;
  sfloat* wcdof = (sfloat*)c.hwin();
  sfloat* wqvel = wcdof + 6 * m.nv;
  sfloat* wscom = wqvel + m.nv;
  sint* wchain = (sint*)(wscom + 3 * m.nbody);
  wave_copy2(wcdof, c.F(c.L().cdof), 6 * m.nv, wchain, c.ni() + c.I().chain, chainw * m.nbody, c.lane());
  wave_copy2(wqvel, qvel, m.nv, wscom, c.F(c.L().scom), 3 * m.nbody, c.lane());
  sync();
  auto chain_of = [&](int b) { return wchain + chainw * b; };
  const sfloat* cdof = wcdof;
  const sfloat* scom = wscom;
  const sfloat* qv = wqvel;
#else
  auto chain_of = [&](int b) { return c.chain(b); };
  const real* cdof = c.F(c.L().cdof);
  const real* scom = c.F(c.L().scom);
  const real* qv = qvel;
#endif
  for (int base = 0; base < ncon; base += kLanes) {
    int con = base + c.lane();
    int cnt = 0, dim = 0, g1 = 0, g2 = 0;
    real position = 0.f;
    if (con < ncon) {   // the contact's scalars, loaded together
      const real cd = c.F(c.L().cdist)[con], cm = c.F(c.L().cmargin)[con];
      dim = c.N(c.L().cdim)[con];
      g1 = c.N(c.L().cgeom)[2 * con];
      g2 = c.N(c.L().cgeom)[2 * con + 1];
      position = cd - cm;
      if (position < 0.f) cnt = (m.opt_cone == 1 || dim == 1) ? dim : 2 * (dim - 1);
    }
    int total;
    int off = wave_excl_scan(cnt, c.lane(), total);
    int adr = nr + off;
    bool fits = cnt > 0 && adr + cnt <= R;
    if (con < ncon) c.N(c.L().caddr)[con] = fits ? adr : -1;
    if (cnt > 0 && !fits) ovf = 1;
    if (fits) {
      // contact-frame Jacobian over the union of the two bodies' dof chains (merge of two
      // descending lists); J = jac(body2) - jac(body1) at the contact point
      int b1 = c.gi(g1, G_BODY), b2 = c.gi(g2, G_BODY);
      const real* pos = c.F(c.L().cpos) + 3 * con;
      const real* fr = c.F(c.L().cframe) + 9 * con;
      const real* f5 = c.F(c.L().cfric) + 5 * con;
      const real* sref = c.F(c.L().csolref) + 2 * con;
      const real* simp = c.F(c.L().csolimp) + 5 * con;
      // condim is 1 or 3 (the model compiler rejects others): at most four rows, friction f5[0..1]
      real p3[3] = {pos[0], pos[1], pos[2]}, mu[2] = {f5[0], f5[1]};
      // the frame in registers: the Jacobian's stores below may alias it as far as the compiler
      // knows, which would reload it on every dof
      real f9[9];
#pragma unroll
      for (int k = 0; k < 9; ++k) f9[k] = fr[k];
      real ref[2] = {sref[0], sref[1]}, imp[5] = {simp[0], simp[1], simp[2], simp[3], simp[4]};
      const auto* ch1 = chain_of(b1);
      const auto* ch2 = chain_of(b2);
      int r1 = c.bi(b1, B_ROOT), r2 = c.bi(b2, B_ROOT);
      real weight = c.bf(b1, B_INVW)[0] + c.bf(b2, B_INVW)[0];
      real o1[3] = {p3[0] - scom[3 * r1], p3[1] - scom[3 * r1 + 1], p3[2] - scom[3 * r1 + 2]};
      real o2[3] = {p3[0] - scom[3 * r2], p3[1] - scom[3 * r2 + 1], p3[2] - scom[3 * r2 + 2]};
      int* idx = c.N(c.L().cjidx) + K * con;
      real* jv = c.F(c.L().cjval) + 3 * K * con;
      int i1 = 1, i2 = 1, n1 = ch1[0], n2 = ch2[0], nn = 0;
      real vel[3] = {0.f, 0.f, 0.f};
      while ((i1 <= n1 || i2 <= n2) && nn < K) {
        int d1 = i1 <= n1 ? ch1[i1] : -1, d2 = i2 <= n2 ? ch2[i2] : -1;
        int d = max(d1, d2);
        real lin[3] = {0.f, 0.f, 0.f}, t[3], cd[6];
        for (int k = 0; k < 6; ++k) cd[k] = cdof[6 * d + k];
        if (d == d2) {
          cross3(cd, o2, t);
          for (int k = 0; k < 3; ++k) lin[k] += cd[3 + k] + t[k];
          ++i2;
        }
        if (d == d1) {
          cross3(cd, o1, t);
          for (int k = 0; k < 3; ++k) lin[k] -= cd[3 + k] + t[k];
          ++i1;
        }
        idx[nn] = d;
        const real qd = qv[d];
        for (int a = 0; a < 3; ++a) {
          real v = dot3f(lin, f9 + 3 * a);
          jv[a * K + nn] = v;
          vel[a] += v * qd;
        }
        ++nn;
      }
      c.N(c.L().cjn)[con] = nn;
      // the impedance depends on the contact only: once for its rows
      const KBI kbi = impedance(m.opt_timestep, ref, imp, position);
      for (int comp = 0; comp < cnt; ++comp) {
        int r = adr + comp;
        rid[r] = con;
        // row coefficients on the (normal, tangent1, tangent2) rows
        real co[3];
        if (m.opt_cone == 1 || dim == 1) {
          co[0] = comp == 0 ? 1.f : 0.f;
          co[1] = comp == 1 ? 1.f : 0.f;
          co[2] = comp == 2 ? 1.f : 0.f;
        } else {
          int dir = comp / 2 + 1;
          real f = (dir == 1 ? mu[0] : mu[1]) * (1.f - 2.f * real(comp & 1));
          co[0] = 1.f;
          co[1] = dir == 1 ? f : 0.f;
          co[2] = dir == 2 ? f : 0.f;
        }
        real v = co[0] * vel[0] + co[1] * vel[1] + co[2] * vel[2];
        real wgt = weight, pos_aref = position, scale = 1.f;
        if (m.opt_cone == 1 && comp > 0) {
          scale = ratio2;
          if (comp > 1) scale *= mu[0] * mu[0] / (mu[1] * mu[1]);
          pos_aref = 0.f;
        } else if (m.opt_cone == 0 && dim > 1) {
          wgt = wgt + mu[0] * mu[0] * wgt;
          wgt = wgt * 2.f * mu[0] * mu[0] * ratio2;
        }
        real D = 1.f / r_max(wgt * (1.f - kbi.imp) / kbi.imp, 1e-15f);
        real aref = -kbi.k * kbi.imp * pos_aref - kbi.b * v;
        if (m.opt_cone == 1 && comp > 0) {
          D /= scale;
          aref = -kbi.b * v;
        }
        c.F(c.L().rD)[r] = D;
        c.F(c.L().raref)[r] = aref;
      }
    }
    nr += total;
    if (nr > R) nr = R;
  }
  ovf = __any(ovf);
  if (c.lane() == 0) {
    sv[SV_NEFC] = nr;
    sv[SV_NF] = nf;
    sv[SV_NL] = nl;
    if (ovf) sv[SV_OVF] |= MX_OVERFLOW_NEFC;
  }
  sync();
}

// Packed entry e of the island blocks -> island | row << 8 | column << 18 (row >= column);
// -1 past the end.
template <class IP>
__device__ __forceinline__ int hdecode(const IP* iblk, int nisl, int e, int total) {
  if (e >= total) return -1;
  int I = 0;
  while (I + 1 < nisl && e >= iblk[I + 1]) ++I;
  int t = e - iblk[I];
  int li = (int)((r_sqrt(8.f * (float)t + 1.f) - 1.f) * 0.5f);
  while (li * (li + 1) / 2 > t) --li;
  while ((li + 1) * (li + 2) / 2 <= t) ++li;
  return I | (li << 8) | ((t - li * (li + 1) / 2) << 18);
}

// Islands: trees joined by contact rows (union-find by one lane).  Each island's Hessian is a
// dense block (packed lower triangle); trees in island order, dofs of a tree consecutive.
__device__ void islands(const Ctx& c) {
  KModel& m = c.m();
  int* sv = c.SV();
  int* tisl = c.N(c.L().tisl);
  int* isz = c.N(c.L().isz);
  int* toff = c.N(c.L().toff);   // first island-local dof of each tree
  int* iblk = c.N(c.L().iblk);
  int* istart = c.N(c.L().istart);
  const int nt = m.ntree;
#ifdef MX_SLAB
  // The union-find runs on LDS copies in the window (free at this point): the lanes first read
  // each contact's two trees and the trees' dof counts in parallel; the tables go back to the
  // workspace afterwards.
  const int ncon = sv[SV_NCON];
  sint* uf = (sint*)c.hwin();     // parent pointers
  sint* tdn = uf + nt;            // dofs per tree
  sint* ltisl = tdn + nt;         // tree -> island
  sint* ltoff = ltisl + nt;
  sint* lisz = ltoff + nt;
  sint* liblk = lisz + nt;        // nt + 1
  sint* listart = liblk + nt + 1; // nt + 1
  sint* ctr = listart + nt + 1;   // each contact's two trees (-1: contact without rows)
  sint* ldisl = ctr + 2 * ncon;   // dof -> island, island-local index
  sint* ldloc = ldisl + m.nv;
  for (int t = c.lane(); t < nt; t += kLanes) { uf[t] = t; tdn[t] = c.ti(t, T_DOFNUM); }
  for (int con = c.lane(); con < ncon; con += kLanes) {
    int t1 = -1, t2 = -1;
    if (c.N(c.L().caddr)[con] >= 0) {
      t1 = c.bi(c.gi(c.N(c.L().cgeom)[2 * con], G_BODY), B_TREE);
      t2 = c.bi(c.gi(c.N(c.L().cgeom)[2 * con + 1], G_BODY), B_TREE);
    }
    ctr[2 * con] = t1;
    ctr[2 * con + 1] = t2;
  }
  sync();
  // Every table below is a function of this list alone (the union-find's partition of the trees,
  // the tree order numbering the islands): when each contact joins the same two trees as in the
  // substep the tables were built for (same count and order, kept in ctrp), they still hold.
  int* prev = c.N(c.L().ctrp);
  if (sv[SV_ISLAND]) {
    bool diff = prev[0] != ncon;
    for (int t = c.lane(); t < 2 * ncon; t += kLanes) diff |= prev[1 + t] != ctr[t];
    if (!__any(diff)) return;
  }
  for (int t = c.lane(); t < 2 * ncon; t += kLanes) prev[1 + t] = ctr[t];
  if (c.lane() == 0) {
    prev[0] = ncon;
    sv[SV_ISLAND] = 1;
  }
  if (c.lane() == 0) {
    auto find = [&](int x) { while (uf[x] != x) { uf[x] = uf[uf[x]]; x = uf[x]; } return x; };
    for (int con = 0; con < ncon; ++con) {
      int t1 = ctr[2 * con], t2 = ctr[2 * con + 1];
      if (t1 >= 0 && t2 >= 0) {
        int a = find(t1), b = find(t2);
        if (a != b) uf[a > b ? a : b] = a < b ? a : b;
      }
    }
    int nisl = 0;
    for (int t = 0; t < nt; ++t) {
      int r = find(t);
      ltisl[t] = r == t ? nisl++ : ltisl[r];
    }
    for (int i = 0; i < nisl; ++i) lisz[i] = 0;
    for (int t = 0; t < nt; ++t) {
      int I = ltisl[t];
      ltoff[t] = lisz[I];
      lisz[I] += tdn[t];
    }
    int at = 0, maxn = 0, st = 0;
    for (int i = 0; i < nisl; ++i) {
      liblk[i] = at; at += lisz[i] * (lisz[i] + 1) / 2; maxn = max(maxn, lisz[i]);
      listart[i] = st; st += lisz[i];
    }
    liblk[nisl] = at;
    listart[nisl] = st;
    sv[SV_NISL] = nisl;
    sv[SV_MAXISL] = maxn;
  }
  sync();
  const int nisl = sv[SV_NISL];
  for (int t = c.lane(); t < nt; t += kLanes) { tisl[t] = ltisl[t]; toff[t] = ltoff[t]; }
  for (int i = c.lane(); i <= nisl; i += kLanes) {
    if (i < nisl) isz[i] = lisz[i];
    iblk[i] = liblk[i];
    istart[i] = listart[i];
  }
  // per-dof island tables, one lane per dof
  for (int d = c.lane(); d < m.nv; d += kLanes) {
    int t = c.di(d, D_TREE), I = ltisl[t], li = ltoff[t] + d - c.ti(t, T_DOFADR);
    c.N(c.L().disl)[d] = I;
    c.N(c.L().dloc)[d] = li;
    ldisl[d] = I;
    ldloc[d] = li;
    c.N(c.L().idof)[listart[I] + li] = d;
  }
  sync();
  // the Hessian assembly's mass-entry map and the sweep's per-lane decodes, from the LDS tables:
  // hmap[e] = packed island-block index of mass entry e (-1 above the diagonal)
  const int* ent = c.IN(c.I().mentry);
  int* hmap = c.N(c.L().hmap);
  for (int e = c.lane(); e < m.nM; e += kLanes) {
    int cd = ent[2 * e], i = (cd >> 16) & 63, j = (cd >> 22) & 63;
    int di = ent[2 * e + 1], dj = di - i + j, li = ldloc[di];
    hmap[e] = j > i ? -1 : liblk[ldisl[di]] + li * (li + 1) / 2 + ldloc[dj];
  }
  const int total = liblk[nisl];
  int* own = c.N(c.L().hown);
#pragma unroll
  for (int q = 0; q < kOwn; ++q) {
    int code = hdecode(liblk, nisl, c.lane() + kLanes * q, total), I = code >= 0 ? (code & 255) : 0;
    own[q * kLanes + c.lane()] = code;
    own[(kOwn + q) * kLanes + c.lane()] = code >= 0 ? lisz[I] : 0;
    own[(2 * kOwn + q) * kLanes + c.lane()] = code >= 0 ? listart[I] : 0;
  }
  int sn[4] = {0, 0, 0, 0};
  if (c.lane() < m.nv) {
    int I = ldisl[c.lane()];
    sn[0] = lisz[I]; sn[1] = listart[I] + ldloc[c.lane()]; sn[2] = ldloc[c.lane()]; sn[3] = liblk[I];
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) own[(3 * kOwn + q) * kLanes + c.lane()] = sn[q];
  sync();
#else
  if (c.lane() == 0) {
    int* uf = iblk;   // scratch: parent pointers
    for (int t = 0; t < nt; ++t) uf[t] = t;
    auto find = [&](int x) { while (uf[x] != x) { uf[x] = uf[uf[x]]; x = uf[x]; } return x; };
    int ncon = sv[SV_NCON];
    for (int con = 0; con < ncon; ++con) {
      if (c.N(c.L().caddr)[con] < 0) continue;
      int t1 = c.bi(c.gi(c.N(c.L().cgeom)[2 * con], G_BODY), B_TREE);
      int t2 = c.bi(c.gi(c.N(c.L().cgeom)[2 * con + 1], G_BODY), B_TREE);
      if (t1 >= 0 && t2 >= 0) {
        int a = find(t1), b = find(t2);
        if (a != b) uf[a > b ? a : b] = a < b ? a : b;
      }
    }
    int nisl = 0;
    for (int t = 0; t < nt; ++t) {
      int r = find(t);
      tisl[t] = r == t ? nisl++ : tisl[r];
    }
    for (int i = 0; i < nisl; ++i) isz[i] = 0;
    for (int t = 0; t < nt; ++t) {
      int I = tisl[t];
      toff[t] = isz[I];
      isz[I] += c.ti(t, T_DOFNUM);
    }
    int at = 0, maxn = 0, st = 0;
    for (int i = 0; i < nisl; ++i) {
      iblk[i] = at; at += isz[i] * (isz[i] + 1) / 2; maxn = max(maxn, isz[i]);
      istart[i] = st; st += isz[i];
    }
    iblk[nisl] = at;
    istart[nisl] = st;
    sv[SV_NISL] = nisl;
    sv[SV_MAXISL] = maxn;
  }
  sync();
  // per-dof island tables, one lane per dof
  for (int d = c.lane(); d < m.nv; d += kLanes) {
    int t = c.di(d, D_TREE), I = tisl[t], li = toff[t] + d - c.ti(t, T_DOFADR);
    c.N(c.L().disl)[d] = I;
    c.N(c.L().dloc)[d] = li;
    c.N(c.L().idof)[istart[I] + li] = d;
  }
  sync();
#endif
}

// island-ordered dof list is implicit: the dofs of an island are those with disl == I, in dof order
// Double accumulation through an address-space-qualified pointer (ds_add_f64 in LDS,
// global_atomic_add_f64 in device memory): a generic-pointer atomic would take the flat path.
template <class HD>
__device__ __forceinline__ void hadd(HD* p, double v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Packed lower-triangle entry (li, lj), li >= lj, of island I's Hessian block.
template <class HD>
__device__ __forceinline__ HD* hent(HD* H, const int* iblk, int I, int li, int lj) {
  return H + iblk[I] + li * (li + 1) / 2 + lj;
}

// out[r] = J_r . x for every row (contact rows through their frame Jacobian)
// Where a Newton solve keeps its per-substep contact Jacobian (3 K values and K dof indices per
// contact), the Hessian assembly's column maps, the J^T f accumulator and the Hessian island
// blocks with their pivot column: the working set (WsView), or, on the workspace route when they
// fit, the world's LDS window (WinView).  The address spaces are part of the type so that every
// access compiles to LDS or global instructions, never to the flat path.
template <class Fl, class In, class Db, bool kStaged = false, class RF = Fl, class RI = In, class JM = In>
struct NView {
  using F = Fl;
  using D = Db;
  static constexpr bool kStage = kStaged;   // xs: a window vector that dof-indexed reads go through
  const Fl* jval;
  const In* jidx;
  JM* jmap;   // packed island-local index and row base (32-bit)
  Fl* qcon;
  Db* H;
  Db* col;
  Db* q;      // workspace route: 3x3 contact-space Hessian weight per contact
  In* qn;     // workspace route: Jacobian columns per contact (0: contact without rows)
  Fl* xs;     // kStage: nv floats (a copy of the vector a pass gathers by dof index)
  // workspace route: the assembled (unswept) island blocks and the per-contact weight changes of an
  // incremental rebuild, in the window when it has room, else in the world's slab (copied once per
  // rebuild, so a generic pointer serves both)
  double* Hs = nullptr;
  double* dq = nullptr;
  // the rows (id, D, aref, J qacc - aref, J search, force, state) and the contacts' row address,
  // dim, Jacobian column count, contact-frame product and friction: the working set's arrays, or
  // copies in the window when it has room for them with the Jacobian
  RI* rid;
  RF* rD;
  RF* raref;
  RF* rjaref;
  RF* rjv;
  RF* rforce;
  RI* rstate;
  RI* caddr;
  RI* cdim;
  RI* cjn;
  RF* cdot;
  RF* cfric;
  bool copied = false;   // rows and contacts are window copies (forces and states written back)
};
// The window views keep the Jacobian's dof indices, the per-contact column counts and the copied
// rows' and contacts' integers (row ids and their single-dof codes, states, row addresses, dims,
// column counts) as 16-bit values, all of which fit; the half-size copies leave room for the whole
// solve in the window for worlds a few contacts or island entries larger.
using WsView = NView<lreal, lint, ldouble>;
using WinView = NView<sfloat, sshort, sdouble, true, sfloat, sshort, sint>;  // rows and contacts copied too
using WinJView = NView<sfloat, sshort, sdouble, true, lfloat, lint, sint>;   // the Jacobian, blocks and vectors
using HWinView = NView<lfloat, lint, sdouble>;   // only the island blocks in the window

// the rows' and contacts' arrays of a view: the working set's
template <class V>
__device__ __forceinline__ void working_set_rows(const Ctx& c, V& v) {
  v.rid = c.n() + c.L().rid; v.rD = c.R(c.L().rD); v.raref = c.R(c.L().raref);
  v.rjaref = c.R(c.L().rjaref); v.rjv = c.R(c.L().rjv); v.rforce = c.R(c.L().rforce);
  v.rstate = c.n() + c.L().rstate; v.caddr = c.n() + c.L().caddr; v.cdim = c.n() + c.L().cdim;
  v.cjn = c.n() + c.L().cjn; v.cdot = c.R(c.L().cdot); v.cfric = c.R(c.L().cfric);
}

template <class V, class OP>
__device__ void rows_dot(const Ctx& c, const V& v, const real* x, OP* out) {
  KModel& m = c.m();
  const int ncon = c.SV()[SV_NCON], nefc = c.SV()[SV_NEFC], K = m.maxpairdof;
  if constexpr (V::kStage) {   // x gathered by dof index below: one coalesced copy into the window
    for (int i = c.lane(); i < m.nv; i += kLanes) v.xs[i] = x[i];
    sync();
  }
  for (int con = c.lane(); con < ncon; con += kLanes) {
    if (v.caddr[con] < 0) continue;
    const auto* idx = v.jidx + K * con;
    const auto* jv = v.jval + 3 * K * con;
    int nn = v.cjn[con];
    real s0 = 0.f, s1 = 0.f, s2 = 0.f;
    for (int k = 0; k < nn; ++k) {
      real xv;
      if constexpr (V::kStage) xv = v.xs[idx[k]];
      else xv = x[idx[k]];
      s0 += jv[k] * xv; s1 += jv[K + k] * xv; s2 += jv[2 * K + k] * xv;
    }
    auto* cd = v.cdot + 3 * con;
    cd[0] = s0; cd[1] = s1; cd[2] = s2;
  }
  sync();
  for (int r = c.lane(); r < nefc; r += kLanes) {
    int id = v.rid[r];
    real val;
    if (id >= 0) {
      real co[3];
      row_coef(m, v.cdim, v.cfric, id, r - v.caddr[id], co);
      const auto* cd = v.cdot + 3 * id;
      val = co[0] * cd[0] + co[1] * cd[1] + co[2] * cd[2];
    } else {
      real sign;
      int kind;
      int d = single_dof(id, sign, kind);
      val = sign * x[d];
    }
    out[r] = val;
  }
  sync();
}

__device__ __forceinline__ real safe_div(real x, real y) { return x / (y != 0.f ? y : 1e-15f); }

// Rows whose quadratic state flipped in the last gradient call that asked for them, in the world's
// scalar slots: row r is bit r % 64 of word r / 64 (rows below kFlipRows), each word as two ints
// from SV_FLIP on; SV_FLIPOK is 0 when the summary does not apply (more rows, or a row in the
// elliptic cone state before or after the call), and then every row counts as flipped.
constexpr int kFlipRows = 256;
__device__ __forceinline__ unsigned long long flip_word(const int* sv, int k) {
  return (unsigned long long)(unsigned)sv[SV_FLIP + 2 * k] | ((unsigned long long)(unsigned)sv[SV_FLIP + 2 * k + 1] << 32);
}
__device__ __forceinline__ bool flip_bit(const int* sv, int r) {
  return !sv[SV_FLIPOK] || (r < kFlipRows && ((flip_word(sv, r >> 6) >> (r & 63)) & 1ull));
}

// Row forces/states (constraint_gradient, mjwarp_constraint.cu:107-201), qfrc_constraint = J^T f
// and grad = Ma - qfrc_smooth - qfrc_constraint; returns ||grad||^2 (uniform).
// *hchanged (when given): whether any row changed state (or is in the cone state, whose curvature
// follows jaref) since the previous call, i.e. whether the Hessian must be rebuilt.
// flips: record the rows whose state entered or left QUADRATIC, the only state property a
// pyramidal-cone Hessian depends on (flip_word / flip_bit read them after the call).
template <class V>
__device__ real gradient(const Ctx& c, const V& v, bool* hchanged = nullptr, bool flips = false) {
  KModel& m = c.m();
  const int ncon = c.SV()[SV_NCON], nefc = c.SV()[SV_NEFC], K = m.maxpairdof;
  const int nfr = c.SV()[SV_NF];
  const auto* rid = v.rid;
  const auto* D = v.rD;
  const auto* jaref = v.rjaref;
  auto* force = v.rforce;
  auto* state = v.rstate;
  const real ratio = 1.f / r_sqrt(m.opt_impratio);
  bool changed = false, cone = false;
  unsigned fbits = 0u;   // bit k: this lane's row 64 k + lane flipped
  for (int r = c.lane(); r < nefc; r += kLanes) {
    real d = D[r], res = jaref[r], f;
    int st;
    int id = rid[r];
    if (r < nfr) {
      real sign;
      int kind;
      int dof = single_dof(id, sign, kind);
      real loss = c.df(dof, D_FLOSS), rad = safe_div(loss, d);
      if (res <= -rad) { f = loss; st = ST_LINEAR_NEG; }
      else if (res >= rad) { f = -loss; st = ST_LINEAR_POS; }
      else { f = -d * res; st = ST_QUADRATIC; }
    } else if (id >= 0 && m.opt_cone == 1 && v.cdim[id] > 1) {
      int head = v.caddr[id], dim = v.cdim[id];
      const auto* fr = v.cfric + 5 * id;
      real mu = fr[0] * ratio, normal = jaref[head], d0 = D[head], tt = 0.f, ts = 0.f;
      for (int j = 1; j < dim; ++j) {
        real u = jaref[head + j] * fr[j - 1];
        tt += u * u;
        if (r == head + j) ts = u * fr[j - 1];
      }
      real n = normal * mu, t = tt <= 0.f ? 0.f : r_sqrt(tt);
      if (n >= mu * t || (t <= 0.f && n >= 0.f)) { f = 0.f; st = ST_SATISFIED; }
      else if (mu * n + t <= 0.f || (t <= 0.f && n < 0.f)) { f = -d * res; st = ST_QUADRATIC; }
      else {
        real dm = safe_div(d0, mu * mu * (1.f + mu * mu));
        real fn = -dm * (n - mu * t) * mu;
        f = r == head ? fn : -safe_div(fn, t) * ts;
        st = ST_CONE;
      }
    } else if (res >= 0.f) { f = 0.f; st = ST_SATISFIED; }
    else { f = -d * res; st = ST_QUADRATIC; }
    force[r] = f;
    const int old = state[r];
    changed |= old != st || st == ST_CONE;
    if ((old == ST_QUADRATIC) != (st == ST_QUADRATIC) && r < kFlipRows) fbits |= 1u << (r / kLanes);
    cone |= st == ST_CONE || old == ST_CONE;   // cone curvature entering or leaving the Hessian
    state[r] = st;
  }
  if (hchanged) *hchanged = __ballot(changed) != 0ull;
  if (flips) {   // read after the barrier below
    const bool ok = nefc <= kFlipRows && __ballot(cone) == 0ull;
    int* sv = c.SV();
#pragma unroll
    for (int k = 0; k < kFlipRows / kLanes; ++k) {
      const unsigned long long wk = __ballot((fbits >> k) & 1u);
      if (c.lane() == 0) { sv[SV_FLIP + 2 * k] = (int)(unsigned)wk; sv[SV_FLIP + 2 * k + 1] = (int)(unsigned)(wk >> 32); }
    }
    if (c.lane() == 0) sv[SV_FLIPOK] = ok;
  }
  auto* qcon = v.qcon;
  for (int i = c.lane(); i < m.nv; i += kLanes) qcon[i] = 0.f;
  sync();
  for (int con = c.lane(); con < ncon; con += kLanes) {
    int adr = v.caddr[con];
    if (adr < 0) continue;
    int dim = v.cdim[con];
    int cnt = (m.opt_cone == 1 || dim == 1) ? dim : 2 * (dim - 1);
    real fc[3] = {0.f, 0.f, 0.f};
    for (int comp = 0; comp < cnt; ++comp) {
      real co[3];
      row_coef(m, v.cdim, v.cfric, con, comp, co);
      real fr = force[adr + comp];
      for (int a = 0; a < 3; ++a) fc[a] += co[a] * fr;
    }
    const auto* idx = v.jidx + K * con;
    const auto* jv = v.jval + 3 * K * con;
    int nn = v.cjn[con];
    for (int k = 0; k < nn; ++k)
      __hip_atomic_fetch_add(qcon + idx[k], fc[0] * jv[k] + fc[1] * jv[K + k] + fc[2] * jv[2 * K + k],
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  for (int r = c.lane(); r < nefc; r += kLanes) {
    int id = rid[r];
    if (id >= 0) continue;
    real sign;
    int kind;
    int dof = single_dof(id, sign, kind);
    __hip_atomic_fetch_add(qcon + dof, sign * force[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  sync();
  real g2 = 0.f;
  for (int i = c.lane(); i < m.nv; i += kLanes) {
    real q = qcon[i];
    real g = c.F(c.L().Ma)[i] - c.F(c.L().smooth)[i] - q;
    c.F(c.L().qcon)[i] = q;                       // qfrc_constraint in the working set
    c.F(c.L().grad)[i] = g;
    g2 += g * g;
  }
  g2 = wave_sum(g2);
  sync();
  return g2;
}

#ifdef MX_SLAB
// Per-substep index maps of the Hessian assembly (the islands and contacts are fixed within a
// substep): hmap[e] = packed island-block index of mass entry e (-1 above the diagonal);
// cjmap[con K + j] = island-local index of Jacobian column j | its packed row base << 10.  They
// replace two or three dependent lookups per entry in every Newton iteration.
template <class V>
__device__ void hessian_maps(const Ctx& c, const V& v) {
  KModel& m = c.m();
  const int* sv = c.SV();
  const int ncon = sv[SV_NCON], K = m.maxpairdof;
  const int* iblk = c.N(c.L().iblk);
  const int* disl = c.N(c.L().disl);
  const int* dloc = c.N(c.L().dloc);
  auto* cjmap = v.jmap;
  const auto* cjidx = v.jidx;
  const auto* cjn = v.cjn;
  for (int t = c.lane(); t < ncon * K; t += kLanes) {
    int con = t / K, k = t - con * K;
    if (k >= cjn[con]) continue;
    int dk = cjidx[t], lk = dloc[dk];
    cjmap[t] = lk | ((iblk[disl[dk]] + lk * (lk + 1) / 2) << 10);
  }
  sync();
}
#endif

// H = M + sum_rows D J^T J (quadratic rows) + elliptic cone curvature, per island block
// (mjwarp_hessian.cu:33-212), then the in-place symmetric sweep inverse of every block.
// 3x3 contact-space weight of contact `con` (rows at adr): sum over its quadratic rows of D c c^T
// (c = the row's coefficients on the contact frame), plus the elliptic cone's curvature.
template <class V>
__device__ __forceinline__ void contact_weight(const Ctx& c, const V& v, int con, int adr, int dim, double* Q) {
  KModel& m = c.m();
  const auto* D = v.rD;
  const auto* state = v.rstate;
  const real ratio = 1.f / r_sqrt(m.opt_impratio);
  int cnt = (m.opt_cone == 1 || dim == 1) ? dim : 2 * (dim - 1);
  for (int i = 0; i < 9; ++i) Q[i] = 0.0;
  // the rows' states and D first (independent loads; condim <= 3 gives at most 4 rows)
  int st[4];
  real dd[4];
#pragma unroll
  for (int comp = 0; comp < 4; ++comp) {
    st[comp] = comp < cnt ? state[adr + comp] : -1;
    dd[comp] = comp < cnt ? D[adr + comp] : 0.f;
  }
#pragma unroll
  for (int comp = 0; comp < 4; ++comp) {
    if (st[comp] != ST_QUADRATIC) continue;
    real co[3];
    row_coef(m, v.cdim, v.cfric, con, comp, co);
    double dr = dd[comp];
    for (int a = 0; a < 3; ++a)
      for (int b = 0; b < 3; ++b) Q[3 * a + b] += dr * co[a] * co[b];
  }
  if (m.opt_cone == 1 && dim > 1 && state[adr] == ST_CONE) {
    const auto* fr = v.cfric + 5 * con;
    const auto* jaref = v.rjaref;
    real mu = fr[0] * ratio, mu2 = mu * mu, den = mu2 * (1.f + mu2);
    real dm = D[adr] / (den != 0.f ? den : 1e-15f);
    real n = jaref[adr] * mu, tt = 0.f, u[3] = {0.f, 0.f, 0.f};
    // fixed trip counts with guards keep u, p and Q in registers (condim <= 3)
#pragma unroll
    for (int d = 1; d < 3; ++d)
      if (d < dim) { u[d] = jaref[adr + d] * fr[d - 1]; tt += u[d] * u[d]; }
    real tl = r_max(r_sqrt(tt), 1e-15f), it = 1.f / tl, mnt = mu * n * it;
    real p[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 1; d < 3; ++d)
      if (d < dim) p[d] = u[d] * fr[d - 1] * it;
    Q[0] += dm * mu2;
#pragma unroll
    for (int d = 1; d < 3; ++d) {
      if (d >= dim) continue;
      Q[d] += dm * (-mu * mu * p[d]);
      Q[3 * d] += dm * (-mu * mu * p[d]);
#pragma unroll
      for (int e = 1; e < 3; ++e)
        if (e < dim) Q[3 * d + e] += dm * mnt * p[d] * p[e];
      Q[4 * d] += dm * (mu2 - mnt) * fr[d - 1] * fr[d - 1];
    }
  }
}

// H and col: the island blocks and the pivot column, in the working set or in an LDS window.
// incremental (workspace route, v.Hs set): the blocks are rebuilt from the saved assembly by
// re-adding only what the rows whose quadratic state flipped (flip_bit) contribute.
template <class V>
__device__ void hessian_inverse(const Ctx& c, const V& v, bool incremental = false) {
  using HD = typename V::D;
  HD* H = v.H;
  HD* col = v.col;
  KModel& m = c.m();
  const int* sv = c.SV();
  const int ncon = sv[SV_NCON], nefc = sv[SV_NEFC], K = m.maxpairdof, nisl = sv[SV_NISL];
  const int* iblk = c.N(c.L().iblk);
  const int* disl = c.N(c.L().disl);
  const int* dloc = c.N(c.L().dloc);
  const int* istart = c.N(c.L().istart);
  const int* isz = c.N(c.L().isz);
  const int maxn = sv[SV_MAXISL], total = iblk[nisl];
  const auto* D = v.rD;
  const auto* state = v.rstate;
  const auto* rid = v.rid;
  int own[kOwn], own_n[kOwn], own_col[kOwn];
  // per-lane constants of the column snapshot (one dof per lane while nv <= 64)
  int sn_n = 0, sn_col = 0, sn_li = 0, sn_blk = 0;
#ifdef MX_SLAB
  {   // decoded once per substep by hessian_maps
    const int* cache = c.N(c.L().hown);
#pragma unroll
    for (int q = 0; q < kOwn; ++q) {
      own[q] = cache[q * kLanes + c.lane()];
      own_n[q] = cache[(kOwn + q) * kLanes + c.lane()];
      own_col[q] = cache[(2 * kOwn + q) * kLanes + c.lane()];
    }
    sn_n = cache[3 * kOwn * kLanes + c.lane()];
    sn_col = cache[(3 * kOwn + 1) * kLanes + c.lane()];
    sn_li = cache[(3 * kOwn + 2) * kLanes + c.lane()];
    sn_blk = cache[(3 * kOwn + 3) * kLanes + c.lane()];
  }
  // K entries of column k of contact con's J^T Q J (Q: 3x3 from Qsrc), added into the blocks Hdst;
  // one lane per (contact, column k) over the columns of the contacts with qn > 0 only (their
  // count prefix-summed over the contacts, one contact per lane, and each item's contact found by
  // a binary search over the lanes' sums)
  auto columns = [&](const auto* Qsrc, HD* Hdst) {
    const bool packed = ncon <= kLanes;
    const int myn = packed && c.lane() < ncon ? v.qn[c.lane()] : 0;
    const int incl = wave_incl_scan(myn), excl = incl - myn;
    const int items = packed ? __builtin_amdgcn_readlane(incl, 63) : ncon * K;
    for (int t0 = 0; t0 < items; t0 += kLanes) {
      const int t = t0 + c.lane();
      int con, k, nn;
      if (packed) {
        int lo = 0;
#pragma unroll
        for (int step = 32; step >= 1; step >>= 1)
          if (__shfl(incl, lo + step - 1) <= t) lo += step;
        con = lo;
        k = t - __shfl(excl, lo);
        nn = __shfl(myn, lo);
        if (t >= items) continue;
      } else {
        if (t >= items) continue;
        con = t / K; k = t % K; nn = v.qn[con];
        if (k >= nn) continue;
      }
      const auto* Qv = Qsrc + 9 * con;
      const auto* jv = v.jval + 3 * K * con;
      double uk[3];
      for (int a = 0; a < 3; ++a)
        uk[a] = Qv[3 * a] * jv[k] + Qv[3 * a + 1] * (double)jv[K + k] + Qv[3 * a + 2] * (double)jv[2 * K + k];
      const auto* cjm = v.jmap + K * con;
      const int mk = cjm[k], lk = mk & 1023;
      HD* Hrow = Hdst + (mk >> 10);                  // row lk of its island (packed lower)
      // columns in chunks of four: the chunk's loads are issued together, then its updates
      for (int j0 = 0; j0 < nn; j0 += 4) {
        int lq[4];
        real a0[4], a1[4], a2[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          int j = j0 + q < nn ? j0 + q : j0;
          lq[q] = cjm[j] & 1023;
          a0[q] = jv[j]; a1[q] = jv[K + j]; a2[q] = jv[2 * K + j];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          double hv = uk[0] * a0[q] + uk[1] * (double)a1[q] + uk[2] * (double)a2[q];
          if (j0 + q < nn && lq[q] <= lk) hadd(Hrow + lq[q], hv);
        }
      }
    }
  };
  if (incremental) {
    // contacts with a flipped row: new weight, its change from the saved one
    for (int con = c.lane(); con < ncon; con += kLanes) {
      int adr = v.caddr[con], nn0 = v.cjn[con], dim = v.cdim[con];
      int cnt = (m.opt_cone == 1 || dim == 1) ? dim : 2 * (dim - 1);
      bool hit = false;
      for (int q = 0; adr >= 0 && q < cnt; ++q) hit |= flip_bit(c.SV(), adr + q);
      if (hit) {
        double Q[9];
        contact_weight(c, v, con, adr, dim, Q);
#pragma unroll
        for (int i = 0; i < 9; ++i) { v.dq[9 * con + i] = Q[i] - v.q[9 * con + i]; v.q[9 * con + i] = Q[i]; }
      }
      v.qn[con] = hit ? nn0 : 0;
    }
    // the saved assembly into the blocks, the changes added there, the result saved again (the
    // sweep below reads every entry before its first update, behind a barrier)
    for (int e = c.lane(); e < total; e += kLanes) H[e] = v.Hs[e];
    sync();
    columns(v.dq, H);
    for (int r = c.lane(); r < nefc; r += kLanes) {
      int id = rid[r];
      if (id >= 0 || !flip_bit(c.SV(), r)) continue;
      real sign;
      int kind;
      int dof = single_dof(id, sign, kind);
      double dd = state[r] == ST_QUADRATIC ? (double)D[r] : -(double)D[r];
      hadd(hent(H, iblk, disl[dof], dloc[dof], dloc[dof]), dd);
    }
    sync();
    for (int e = c.lane(); e < total; e += kLanes) v.Hs[e] = H[e];
  } else {
#endif
  for (int e = c.lane(); e < iblk[nisl]; e += kLanes) H[e] = 0.0;
  sync();
  // mass blocks (lower triangles of each tree block)
#ifdef MX_SLAB
  const int* hmap = c.N(c.L().hmap);
  const real* Mf = c.F(c.L().M);
  for (int e0 = c.lane(); e0 < m.nM; e0 += kBatch * kLanes) {   // loads of kBatch entries issue together
    int h[kBatch];
    real v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      int e = e0 + u * kLanes < m.nM ? e0 + u * kLanes : e0;
      h[u] = hmap[e];
      v[u] = Mf[e];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (e0 + u * kLanes < m.nM && h[u] >= 0) H[h[u]] = (double)v[u];
  }
#else
  const int* ent = c.IN(c.I().mentry);
  for (int e = c.lane(); e < m.nM; e += kLanes) {
    int cd = ent[2 * e], i = (cd >> 16) & 63, j = (cd >> 22) & 63;
    if (j > i) continue;
    int di = ent[2 * e + 1], dj = di - i + j;
    *hent(H, iblk, disl[di], dloc[di], dloc[dj]) = (double)c.F(c.L().M)[e];
  }
#endif
  sync();
#ifdef MX_SLAB
  // contacts: first one lane per contact for its 3x3 weight Q and column count, then one lane per
  // (contact, column k) for the K entries of column k, reading Q from the view
  for (int con = c.lane(); con < ncon; con += kLanes) {
    int adr = v.caddr[con], nn0 = v.cjn[con], dim = v.cdim[con];
    double Q[9];
    if (adr >= 0) contact_weight(c, v, con, adr, dim, Q);
#pragma unroll
    for (int i = 0; i < 9; ++i) v.q[9 * con + i] = adr >= 0 ? Q[i] : 0.0;
    v.qn[con] = adr < 0 ? 0 : nn0;
  }
  sync();
  columns(v.q, H);
#else
  // contacts: lane per (contact, column k); 3x3 contact-space weight Q, then K entries of column k
  for (int t = c.lane(); t < ncon * K; t += kLanes) {
    int con = t / K, k = t % K;
    int adr = v.caddr[con], nn0 = v.cjn[con], dim = v.cdim[con];
    if (adr < 0 || k >= nn0) continue;
    double Q[9];
    contact_weight(c, v, con, adr, dim, Q);
    const auto* idx = v.jidx + K * con;
    const auto* jv = v.jval + 3 * K * con;
    int nn = nn0;
    double uk[3];
    for (int a = 0; a < 3; ++a)
      uk[a] = Q[3 * a] * jv[k] + Q[3 * a + 1] * (double)jv[K + k] + Q[3 * a + 2] * (double)jv[2 * K + k];
    int dk = idx[k], I = disl[dk], lk = dloc[dk];
    HD* Hrow = H + iblk[I] + lk * (lk + 1) / 2;   // row lk of island I (packed lower)
    for (int j = 0; j < nn; ++j) {
      int lj = dloc[idx[j]];
      double hv = uk[0] * jv[j] + uk[1] * (double)jv[K + j] + uk[2] * (double)jv[2 * K + j];
      if (lj <= lk) hadd(Hrow + lj, hv);
    }
  }
#endif
  for (int r = c.lane(); r < nefc; r += kLanes) {
    int id = rid[r];
    if (id >= 0 || state[r] != ST_QUADRATIC) continue;
    real sign;
    int kind;
    int dof = single_dof(id, sign, kind);
    hadd(hent(H, iblk, disl[dof], dloc[dof], dloc[dof]), (double)D[r]);
  }
  sync();
#ifdef MX_SLAB
  if (v.Hs) {   // the assembly, saved for incremental rebuilds within this substep
    for (int e = c.lane(); e < iblk[nisl]; e += kLanes) v.Hs[e] = H[e];
    sync();
  }
  }
#endif
  // symmetric sweep of every island block in place: after all pivots the block holds -H^-1.
  // step k: p = a_kk; a_ij -= (a_ik / p) a_jk (i, j != k); a_ik /= p; a_kk = -1/p.  Column k of
  // every island is saved first (island-local order, the pivot saved as its reciprocal 1/p, one
  // division per island and step), then the packed entries of all blocks are updated in parallel,
  // each lane owning the entries lane, lane + 64, ...
#ifndef MX_SLAB
#pragma unroll
  for (int q = 0; q < kOwn; ++q) own[q] = hdecode(iblk, nisl, c.lane() + kLanes * q, total);
  if (c.lane() < m.nv) {
    int I = disl[c.lane()];
    sn_li = dloc[c.lane()]; sn_n = isz[I]; sn_col = istart[I] + sn_li; sn_blk = iblk[I];
  }
#pragma unroll
  for (int q = 0; q < kOwn; ++q) {
    int I = own[q] >= 0 ? (own[q] & 255) : 0;
    own_n[q] = own[q] >= 0 ? isz[I] : 0;
    own_col[q] = own[q] >= 0 ? istart[I] : 0;
  }
#endif
  for (int k = 0; k < maxn; ++k) {
    if (c.lane() < m.nv) {
      if (k < sn_n) {
        int hi = max(sn_li, k), lo = min(sn_li, k);
        double hv = H[sn_blk + hi * (hi + 1) / 2 + lo];
        col[sn_col] = sn_li == k ? 1.0 / hv : hv;
      }
    } 
    for (int d = c.lane() + kLanes; d < m.nv; d += kLanes) {
      int I = disl[d], li = dloc[d];
      if (k < isz[I]) {
        double hv = li >= k ? *hent(H, iblk, I, li, k) : *hent(H, iblk, I, k, li);
        col[istart[I] + li] = li == k ? 1.0 / hv : hv;
      }
    }
    sync();
    auto update = [&](int code, int e, int n, int cst) {
      if (k >= n) return;
      int li = (code >> 8) & 1023, lj = code >> 18;
      const HD* ck = col + cst;
      double inv = ck[k], val;   // the snapshot holds the pivot's reciprocal
      if (li == k) val = lj == k ? -inv : ck[lj] * inv;
      else if (lj == k) val = ck[li] * inv;
      else val = H[e] - (ck[li] * inv) * ck[lj];
      H[e] = val;
    };
#pragma unroll
    for (int q = 0; q < kOwn; ++q)
      if (own[q] >= 0) update(own[q], c.lane() + kLanes * q, own_n[q], own_col[q]);
    for (int e = c.lane() + kLanes * kOwn; e < total; e += kLanes) {
      int code = hdecode(iblk, nisl, e, total), I = code & 255;
      update(code, e, isz[I], istart[I]);
    }
    sync();
  }
}

// Rank-one updates of the swept blocks for rows whose quadratic state flipped (Sherman-Morrison):
// a flipped row r adds delta j j^T to its island's H (delta = +D_r entering QUADRATIC, -D_r leaving
// it; j = the row's Jacobian: its contact-space direction through the contact's 3 x K Jacobian, or
// a unit dof vector), so with G = -H^-1 in the blocks, g = G j and s = j^T g,
//   G' = G + delta g g^T / (1 - delta s).
// Two barriers per row instead of an assembly and a full sweep.  Returns false (blocks untouched
// from the first row on that would divide by a denominator that is not clearly positive) when the
// caller must rebuild from scratch; the caller passes only summaries without cone-state rows.
template <class V>
__device__ __noinline__ bool hessian_rank1(const Ctx& c, const V& v) {
  using HD = typename V::D;
  HD* G = v.H;
  HD* g = v.col;
  KModel& m = c.m();
  const int K = m.maxpairdof, lane = c.lane();
  const int* iblk = c.N(c.L().iblk);
  const int* disl = c.N(c.L().disl);
  const int* dloc = c.N(c.L().dloc);
  const int* istart = c.N(c.L().istart);
  const int* isz = c.N(c.L().isz);
  for (int wk = 0; wk < kFlipRows / kLanes; ++wk)
  for (unsigned long long bits = flip_word(c.SV(), wk); bits; bits &= bits - 1ull) {
    const int r = kLanes * wk + __ffsll((long long)bits) - 1;
    const int id = v.rid[r];
    const double dr = v.rD[r];
    const double delta = v.rstate[r] == ST_QUADRATIC ? dr : -dr;
    // the row's island and its Jacobian, one nonzero per lane k < nn: island-local index and value
    int I, nn = 1, loc = 0;
    double jk = 0.0;
    if (id < 0) {
      real sign;
      int kind;
      const int dof = single_dof(id, sign, kind);
      I = disl[dof];
      loc = dloc[dof];
      jk = lane == 0 ? 1.0 : 0.0;
    } else {
      const int con = id;
      const auto* ji = v.jidx + K * con;
      const auto* jv = v.jval + 3 * K * con;
      I = disl[ji[0]];
      nn = v.cjn[con];
      real co[3];
      row_coef(m, v.cdim, v.cfric, con, r - v.caddr[con], co);
      if (lane < nn) {
        loc = dloc[ji[lane]];
        jk = (double)co[0] * jv[lane] + (double)co[1] * jv[K + lane] + (double)co[2] * jv[2 * K + lane];
      }
    }
    const int n = isz[I], blk = iblk[I], st = istart[I];
    // g = G j, one island dof per lane; the nonzeros come by readlane, G's loads issue four at a time
    for (int a = lane; a < n; a += kLanes) {
      double s = 0.0;
      for (int k0 = 0; k0 < nn; k0 += 4) {
        double gv[4], jv4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int k = k0 + u < nn ? k0 + u : k0;
          const int lk = __shfl(loc, k);
          jv4[u] = __shfl(jk, k);
          gv[u] = *hent(G, iblk, I, max(a, lk), min(a, lk));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (k0 + u < nn) s += gv[u] * jv4[u];
      }
      g[st + a] = s;
    }
    sync();
    // s = j^T g over the nonzeros (lanes k < nn), summed across the wave
    double t = lane < nn ? jk * g[st + loc] : 0.0;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off);
    const double den = 1.0 - delta * t;
    if (!(den > 1e-9)) return false;   // uniform: every lane holds the same sum
    const double f = delta / den;
    // G += f g g^T over the island's packed lower triangle
    const int tri = n * (n + 1) / 2;
    for (int e = lane; e < tri; e += kLanes) {
      int li = (int)((r_sqrt(8.f * e + 1.f) - 1.f) * 0.5f);
      if ((li + 1) * (li + 2) / 2 <= e) ++li;
      if (li * (li + 1) / 2 > e) --li;
      const int lj = e - li * (li + 1) / 2;
      G[blk + e] += f * g[st + li] * g[st + lj];
    }
    sync();
  }
  return true;
}

// A lane's dof and its island (island, local index, size, first island-order slot, block
// address), fixed within a substep: read once per solve when every dof has its own lane.
struct DofIsl { int I, li, n, st, blk; };

__device__ __forceinline__ DofIsl dof_island(const Ctx& c, int d) {
  DofIsl x{0, 0, 0, 0, 0};
  if (d < c.m().nv) {
    x.I = c.N(c.L().disl)[d];
    x.li = c.N(c.L().dloc)[d];
    x.n = c.N(c.L().isz)[x.I];
    x.st = c.N(c.L().istart)[x.I];
    x.blk = c.N(c.L().iblk)[x.I];
  }
  return x;
}

// search = -H^-1 grad (the swept blocks hold -H^-1); returns search.search and grad.H^-1.grad.
// own: the lane's dof island (every dof has its own lane)
template <class V>
__device__ void direction(const Ctx& c, const V& v, const DofIsl& own, real& search_dot, real& decrement) {
  const auto* H = v.H;
  KModel& m = c.m();
  const int* disl = c.N(c.L().disl);
  const int* dloc = c.N(c.L().dloc);
  const int* idof = c.N(c.L().idof);
  const int* istart = c.N(c.L().istart);
  const int* isz = c.N(c.L().isz);
  const real* grad = c.F(c.L().grad);
  real* search = c.F(c.L().search);
  real sd = 0.f, dec = 0.f;
  if (m.nv <= kLanes) {
    const int d = c.lane();
    real gd = d < m.nv ? grad[d] : 0.f;
    if constexpr (V::kStage) {   // the gradient in island order, in the window
      if (d < m.nv) v.xs[own.st + own.li] = gd;
      sync();
    }
    if (d < m.nv) {
      const int li = own.li, n = own.n;
      const auto* Hb = H + own.blk;
      const int* dl = idof + own.st;
      double acc = 0.0;
      for (int lj = 0; lj < n; ++lj) {
        double h = lj <= li ? Hb[li * (li + 1) / 2 + lj] : Hb[lj * (lj + 1) / 2 + li];
        if constexpr (V::kStage) acc += h * (double)v.xs[own.st + lj];
        else acc += h * (double)grad[dl[lj]];
      }
      real s = (real)acc;
      search[d] = s;
      sd += s * s;
      dec -= gd * s;
    }
    search_dot = wave_sum(sd);
    decrement = wave_sum(dec);
    sync();
    return;
  }
  if constexpr (V::kStage) {   // the gradient in island order, in the window
    for (int d = c.lane(); d < m.nv; d += kLanes) v.xs[istart[disl[d]] + dloc[d]] = grad[d];
    sync();
  }
  for (int d = c.lane(); d < m.nv; d += kLanes) {
    int I = disl[d], li = dloc[d], n = isz[I];
    const int* dl = idof + istart[I];
    double acc = 0.0;
    const int* iblk = c.N(c.L().iblk);
    for (int lj = 0; lj < n; ++lj) {
      double h = lj <= li ? *hent(H, iblk, I, li, lj) : *hent(H, iblk, I, lj, li);
      if constexpr (V::kStage) acc += h * (double)v.xs[istart[I] + lj];
      else acc += h * (double)grad[dl[lj]];
    }
    real s = (real)acc;
    search[d] = s;
    sd += s * s;
    dec -= grad[d] * s;
  }
  search_dot = wave_sum(sd);
  decrement = wave_sum(dec);
  sync();
}

// ---- exact line search over the piecewise-quadratic cost (iterative_search,
// gpu/cuda/newton/mjwarp_linesearch.cu:81-375); rows are spread over the lanes and every trial
// point is a wave reduction.
struct LPoint { real cost, slope, curv; };
__device__ __forceinline__ LPoint lp_add(LPoint a, LPoint b) { return {a.cost + b.cost, a.slope + b.slope, a.curv + b.curv}; }
__device__ __forceinline__ LPoint lp_sum(LPoint p) { return {wave_sum(p.cost), wave_sum(p.slope), wave_sum(p.curv)}; }
__device__ __forceinline__ LPoint lp_quadratic(real q1, real q2, real a) {
  real aq2 = a * q2;
  return {a * aq2 + a * q1, 2.f * aq2 + q1, 2.f * q2};
}
__device__ __forceinline__ bool in_bracket(LPoint x, LPoint y) {
  return (x.slope < y.slope && y.slope < 0.f) || (x.slope > y.slope && y.slope > 0.f);
}

struct LRow {
  int kind;   // 0 equality, 1 frictionloss, 2 inequality, 3 primary cone, 4 secondary cone, -1 none
  real x, v, d, loss;
  real q0, q1, q2, u0, v0, uu, uv, vv, dm, mu, cost0, t0, r0;
  int state0;
};

template <class V>
__device__ LRow load_lrow(const Ctx& c, const V& v, int r) {
  LRow x{};
  const int nefc = c.SV()[SV_NEFC], nfr = c.SV()[SV_NF];
  if (r >= nefc) { x.kind = -1; return x; }
  int id = v.rid[r];
  if (r < nfr) x.kind = 1;
  else if (id < 0 || c.m().opt_cone != 1 || v.cdim[id] == 1) x.kind = 2;
  else {
    int head = v.caddr[id];
    if (r != head) { x.kind = 4; return x; }
    x.kind = 3;
    const real* q = c.F(c.L().rquad);
    x.q0 = q[3 * r]; x.q1 = q[3 * r + 1]; x.q2 = q[3 * r + 2];
    x.u0 = q[3 * (r + 1)]; x.v0 = q[3 * (r + 1) + 1]; x.uu = q[3 * (r + 1) + 2];
    x.uv = q[3 * (r + 2)]; x.vv = q[3 * (r + 2) + 1]; x.dm = q[3 * (r + 2) + 2];
    x.mu = v.cfric[5 * id] / r_sqrt(c.m().opt_impratio);
    if (x.uu <= 0.f) { x.state0 = x.u0 < 0.f ? 1 : 0; x.cost0 = x.state0 == 1 ? x.q0 : 0.f; }
    else {
      x.t0 = r_sqrt(x.uu);
      if (x.u0 >= x.mu * x.t0) x.state0 = 0;
      else if (x.mu * x.u0 + x.t0 <= 0.f) { x.state0 = 1; x.cost0 = x.q0; }
      else { x.state0 = 4; x.r0 = x.u0 - x.mu * x.t0; x.cost0 = 0.5f * x.dm * x.r0 * x.r0; }
    }
    return x;
  }
  x.x = v.rjaref[r];
  x.v = v.rjv[r];
  x.d = v.rD[r];
  if (x.kind == 1) {
    real sign;
    int kind;
    x.loss = c.df(single_dof(id, sign, kind), D_FLOSS);
  }
  return x;
}

__device__ __forceinline__ LPoint friction_point(const LRow& r, real x) {
  real rf = safe_div(r.loss, r.d);
  if (-rf < x && x < rf) { real vd = r.v * r.d; return {0.5f * r.d * x * x, vd * x, r.v * vd}; }
  if (x <= -rf) return {r.loss * (-0.5f * rf - x), -r.loss * r.v, 0.f};
  return {r.loss * (-0.5f * rf + x), r.loss * r.v, 0.f};
}

__device__ LPoint eval_zero(const LRow& r) {
  if (r.kind < 0 || r.kind == 4) return {0.f, 0.f, 0.f};
  if (r.kind == 3) {
    if (r.state0 == 1) return {r.q0, r.q1, 2.f * r.q2};
    if (r.state0 == 4) {
      real ti = 1.f / r.t0, t1 = r.uv * ti, t2 = (r.vv - t1 * t1) * ti, r1 = r.v0 - r.mu * t1;
      return {r.cost0, r.dm * r.r0 * r1, r.dm * (r1 * r1 - r.mu * r.r0 * t2)};
    }
    return {0.f, 0.f, 0.f};
  }
  if (r.kind == 1) return friction_point(r, r.x);
  if (r.kind == 2 && r.x >= 0.f) return {0.f, 0.f, 0.f};
  real vd = r.v * r.d;
  return {0.5f * r.d * r.x * r.x, vd * r.x, r.v * vd};
}

__device__ LPoint cone_quadratic_shifted(const LRow& r, real a, real n, real tsqr) {
  real aq2 = a * r.q2, cost = a * (aq2 + r.q1);
  if (r.state0 == 4) { real bd = r.mu * r.u0 + r.t0; cost += 0.5f * r.dm * bd * bd; }
  else if (r.state0 == 0) cost = 0.5f * r.dm * (1.f + r.mu * r.mu) * (n * n + r_max(tsqr, 0.f));
  return {cost, 2.f * aq2 + r.q1, 2.f * r.q2};
}

__device__ LPoint eval_shifted(const LRow& r, real a) {
  if (r.kind < 0 || r.kind == 4) return {0.f, 0.f, 0.f};
  if (r.kind == 3) {
    real n = r.u0 + a * r.v0, tsd = a * (2.f * r.uv + a * r.vv), tsqr = r.uu + tsd;
    if (tsqr <= 0.f) {
      if (n < 0.f) return cone_quadratic_shifted(r, a, n, tsqr);
    } else {
      real t = r_sqrt(tsqr);
      if (n >= r.mu * t) {}
      else if (r.mu * n + t <= 0.f) return cone_quadratic_shifted(r, a, n, tsqr);
      else {
        real ti = 1.f / t, t1 = (r.uv + a * r.vv) * ti, t2 = (r.vv - t1 * t1) * ti;
        real res = n - r.mu * t, r1 = r.v0 - r.mu * t1, cost;
        if (r.state0 == 4) {
          real td = tsd / (t + r.t0), rd = a * r.v0 - r.mu * td;
          cost = 0.5f * r.dm * rd * (2.f * r.r0 + rd);
        } else if (r.state0 == 1) {
          real aq2 = a * r.q2, bd = r.mu * n + t;
          cost = a * (aq2 + r.q1) - 0.5f * r.dm * bd * bd;
        } else cost = 0.5f * r.dm * res * res;
        return {cost, r.dm * res * r1, r.dm * (r1 * r1 + res * (-r.mu * t2))};
      }
    }
    return {-r.cost0, 0.f, 0.f};
  }
  if (r.kind == 1) {
    LPoint p = friction_point(r, r.x + a * r.v);
    p.cost -= friction_point(r, r.x).cost;
    return p;
  }
  real quad0 = 0.5f * r.d * r.x * r.x;
  real cost0 = r.kind == 2 && r.x >= 0.f ? 0.f : quad0;
  if (r.kind == 2 && r.x + a * r.v >= 0.f) return {-cost0, 0.f, 0.f};
  real vd = r.v * r.d, h = r.v * vd, ah = a * h;
  return {a * (vd * r.x + 0.5f * ah) + (quad0 - cost0), vd * r.x + ah, h};
}

// Rows held in registers by one lane during the line search; rows beyond kRowsPerLane * 64 are
// reloaded at every trial point.  The workspace route's 128-register budget holds one (more would
// spill to scratch, which is slower than reloading the rows beyond 64).
#ifdef MX_SLAB
constexpr int kRowsPerLane = 1;
#else
constexpr int kRowsPerLane = 8;
#endif

template <class V>
__device__ real linesearch(const Ctx& c, const V& v, real search_dot, real& improvement, bool& converged) {
  KModel& m = c.m();
  const int nv = m.nv, nefc = c.SV()[SV_NEFC], ncon = c.SV()[SV_NCON];
  const real kNoise = 8.f * 1.1920929e-7f;
  const real* search = c.F(c.L().search);
  real* Mv = c.F(c.L().Mv);
  // Mv = M search, Jv = J search
  for (int i = c.lane(); i < nv; i += kLanes) Mv[i] = block_row_dot(c, c.F(c.L().M), search, i);
  rows_dot(c, v, search, v.rjv);
  if (m.opt_cone == 1) {
    const real ratio = 1.f / r_sqrt(m.opt_impratio);
    real* q = c.F(c.L().rquad);
    const auto* ja = v.rjaref;
    const auto* jv = v.rjv;
    const auto* D = v.rD;
    for (int con = c.lane(); con < ncon; con += kLanes) {
      int at = v.caddr[con], dim = v.cdim[con];
      if (at < 0 || dim == 1) continue;
      const auto* fr = v.cfric + 5 * con;
      real x = ja[at], v = jv[at], d = D[at], vd = v * d;
      real q0 = 0.5f * x * x * d, q1 = vd * x, q2 = 0.5f * v * vd;
      real mu = fr[0] * ratio, u0 = x * mu, v0 = v * mu, uu = 0.f, uv = 0.f, vv = 0.f;
      for (int j = 1; j < dim; ++j) {
        int t = at + j;
        real jvv = jv[t], jaa = ja[t], dj = D[t], djx = dj * jaa;
        q0 += 0.5f * jaa * djx; q1 += jvv * djx; q2 += 0.5f * jvv * dj * jvv;
        real f = fr[j - 1], uj = jaa * f, vj = jvv * f;
        uu += uj * uj; uv += uj * vj; vv += vj * vj;
      }
      q[3 * at] = q0; q[3 * at + 1] = q1; q[3 * at + 2] = q2;
      q[3 * (at + 1)] = u0; q[3 * (at + 1) + 1] = v0; q[3 * (at + 1) + 2] = uu;
      real mu2 = mu * mu;
      q[3 * (at + 2)] = uv; q[3 * (at + 2) + 1] = vv; q[3 * (at + 2) + 2] = d / (mu2 * (1.f + mu2));
    }
    sync();
  }
  const real scale = m.meaninertia * nv;
  const real gtol = r_max(m.opt_tolerance * m.opt_ls_tolerance * r_sqrt(search_dot) * scale, 1e-6f);
  real g1 = 0.f, g2 = 0.f;
  for (int i = c.lane(); i < nv; i += kLanes) {
    g1 += search[i] * (c.F(c.L().Ma)[i] - c.F(c.L().smooth)[i]);
    g2 += 0.5f * search[i] * Mv[i];
  }
  g1 = wave_sum(g1);
  g2 = wave_sum(g2);
  LRow rows[kRowsPerLane];
#pragma unroll
  for (int q = 0; q < kRowsPerLane; ++q) rows[q] = load_lrow(c, v, c.lane() + kLanes * q);
  LPoint local{0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < kRowsPerLane; ++q) local = lp_add(local, eval_zero(rows[q]));
  const int rest = c.lane() + kRowsPerLane * kLanes;
  for (int r = rest; r < nefc; r += kLanes) local = lp_add(local, eval_zero(load_lrow(c, v, r)));
  LPoint rs = lp_sum(local);
  LPoint p0 = lp_add(LPoint{0.f, g1, 2.f * g2}, rs);
  LPoint delta{0.f, p0.slope, p0.curv};
  real q1abs = r_sqrt(2.f * r_max(rs.cost, 0.f) * r_max(rs.curv, 0.f)) + r_abs(g1);
  real gacc = r_max(gtol, kNoise * q1abs), alpha = 0.f;
  improvement = 0.f;
  converged = r_abs(p0.slope) < kNoise * q1abs;
  auto eval = [&](real a) {
    LPoint s{0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < kRowsPerLane; ++q) s = lp_add(s, eval_shifted(rows[q], a));
    for (int r = rest; r < nefc; r += kLanes) s = lp_add(s, eval_shifted(load_lrow(c, v, r), a));
    return lp_add(lp_quadratic(g1, g2, a), lp_sum(s));
  };
  real ia = -safe_div(p0.slope, p0.curv);
  LPoint initial{0.f, 0.f, 0.f};
  if (!converged) {
    initial = eval(ia);
    if (r_abs(initial.slope) < gacc && initial.cost < 0.f) { converged = true; alpha = ia; improvement = -initial.cost; }
  }
  if (!converged) {
    bool less = initial.slope < p0.slope;
    LPoint lo = less ? initial : delta, hi = less ? delta : initial;
    real la = less ? ia : 0.f, ha = less ? 0.f : ia;
    for (int it = 0; it < m.opt_ls_iterations; ++it) {
      real ln = la - safe_div(lo.slope, lo.curv), hn = ha - safe_div(hi.slope, hi.curv), ma = 0.5f * (la + ha);
      LPoint nlo = eval(ln), nhi = eval(hn), mid = eval(ma);
      bool cl = r_abs(nlo.slope) < gacc && nlo.cost < 0.f;
      bool ch = r_abs(nhi.slope) < gacc && nhi.cost < 0.f;
      bool cm = r_abs(mid.slope) < gacc && mid.cost < 0.f;
      bool any = cl || ch || cm, swl = false, swh = false;
      if (any) {
        LPoint best{1e10f, 0.f, 0.f};
        real ba = 0.f;
        if (cl && nlo.cost < best.cost) { best = nlo; ba = ln; }
        if (ch && nhi.cost < best.cost) { best = nhi; ba = hn; }
        if (cm && mid.cost < best.cost) { best = mid; ba = ma; }
        lo = hi = best;
        la = ha = ba;
      } else {
        bool s = in_bracket(lo, nlo);
        if (s) { lo = nlo; la = ln; } swl |= s;
        s = in_bracket(lo, mid);
        if (s) { lo = mid; la = ma; } swl |= s;
        s = in_bracket(lo, nhi);
        if (s) { lo = nhi; la = hn; } swl |= s;
        s = in_bracket(hi, nhi) || (hi.slope < 0.f && nhi.slope > 0.f);
        if (s) { hi = nhi; ha = hn; } swh |= s;
        s = in_bracket(hi, mid);
        if (s) { hi = mid; ha = ma; } swh |= s;
        s = in_bracket(hi, nlo);
        if (s) { hi = nlo; ha = ln; } swh |= s;
      }
      bool done = any || (!swl && !swh) || (lo.cost < 0.f && lo.slope < 0.f && lo.slope > -gtol) ||
                  (hi.cost < 0.f && hi.slope > 0.f && hi.slope < gtol);
      if (lo.cost < 0.f || hi.cost < 0.f) {
        bool bl = lo.cost < hi.cost;
        alpha = bl ? la : ha;
        improvement = -(bl ? lo.cost : hi.cost);
      }
      if (done) { converged = true; break; }
    }
  }
  for (int i = c.lane(); i < nv; i += kLanes) {
    c.F(c.L().qacc)[i] += alpha * search[i];
    c.F(c.L().Ma)[i] += alpha * Mv[i];
  }
  for (int r = c.lane(); r < nefc; r += kLanes) v.rjaref[r] += alpha * v.rjv[r];
  sync();
  return alpha;
}

// The solve proper, on a view of its per-substep arrays.
template <class V>
__device__ void newton_solve(const Ctx& c, const V& v) {
  KModel& m = c.m();
  int* sv = c.SV();
  const int nv = m.nv, nefc = sv[SV_NEFC];
  real* qacc = c.F(c.L().qacc);
#ifdef MX_SLAB
  hessian_maps(c, v);
#endif
  for (int i = c.lane(); i < nv; i += kLanes) c.F(c.L().Ma)[i] = block_row_dot(c, c.F(c.L().M), qacc, i);
  rows_dot(c, v, qacc, v.rjaref);
  for (int r = c.lane(); r < nefc; r += kLanes) v.rjaref[r] -= v.raref[r];
  sync();
  real search_dot, decrement;
  const DofIsl own = dof_island(c, c.lane());
  gradient(c, v);
  hessian_inverse(c, v);
  direction(c, v, own, search_dot, decrement);
  const real scale = m.meaninertia * nv, tol = m.opt_tolerance;
  int niter = 0, ovf = 0;
  bool saved = true;   // the saved assembly (and contact weights) match the blocks' H
  while (m.opt_iterations > 0) {
    real improvement;
    bool ls_ok;
    real alpha = linesearch(c, v, search_dot, improvement, ls_ok);
    if (!ls_ok) ovf |= MX_OVERFLOW_LS_ITERATIONS;
    // the Hessian depends on the rows' states only (and on jaref for cone rows): when none changed,
    // the previous blocks still hold -H^-1
    bool hchanged;
    real grad_dot = gradient(c, v, &hchanged, true);
    const bool fok = sv[SV_FLIPOK] != 0;
    unsigned long long fany = 0ull;
    int fcount = 0;
#pragma unroll
    for (int k = 0; k < kFlipRows / kLanes; ++k) {
      const unsigned long long wk = flip_word(sv, k);
      fany |= wk;
      fcount += __popcll(wk);
    }
    // with the flip summary, no flip means the blocks still hold -H^-1; up to one flipped row per
    // pivot of the largest island updates the blocks by rank-one steps, more rebuild them from the
    // saved assembly when the window holds one (and it is current), else from scratch
    if (hchanged && (!fok || fany != 0ull)) {
      if (fok && fcount <= sv[SV_MAXISL] && hessian_rank1(c, v)) {
        saved = false;
      } else if (fok && v.Hs && saved) {
        hessian_inverse(c, v, true);
      } else {
        hessian_inverse(c, v);
        saved = true;
      }
    }
    direction(c, v, own, search_dot, decrement);
    ++niter;
    real imp = improvement / scale, g = r_sqrt(grad_dot) / scale, mi = 0.5f * decrement / scale;
    bool done = alpha == 0.f || (imp > 0.f && imp < tol) || g < tol || mi < tol;
    if (done || niter == m.opt_iterations) {
      if (!done) ovf |= MX_OVERFLOW_ITERATIONS;
      break;
    }
  }
  if (v.copied)   // the rows' forces and states back to the working set (published, post-constraint)
    for (int r = c.lane(); r < nefc; r += kLanes) {
      c.F(c.L().rforce)[r] = v.rforce[r];
      c.N(c.L().rstate)[r] = v.rstate[r];
    }
  if (c.lane() == 0) { sv[SV_NITER] = niter; sv[SV_OVF] |= ovf; }
  sync();
}

#ifdef MX_SLAB
// Where a view keeps the saved Hessian assembly and the weight changes of incremental rebuilds:
// the window from word `used` when it has room, else the slab's Hessian and contact-weight arrays
// (unused while the blocks and weights live in the window).
template <class V>
__device__ __forceinline__ void saved_assembly(const Ctx& c, V& v, sfloat* wf, int used, int htotal, int ncon) {
  if (used + 2 * htotal + 18 * ncon <= c.L().win) {
    v.Hs = (double*)(sdouble*)(wf + used);
    v.dq = v.Hs + htotal;
  } else {
    v.Hs = (double*)(c.g() + c.L().H);
    v.dq = (double*)(c.g() + c.L().cq);
  }
}
#endif

// Dense Newton with exact line search, world-local (initialize_world mjwarp_solver_state.cu:61-92,
// gradient/Hessian/direction/stopping mjwarp_direction.cu:120-158; the reference's graph WHILE
// over all worlds, runtime.cu:93-131, becomes this per-world loop).
__device__ void newton(const Ctx& c) {
  KModel& m = c.m();
  int* sv = c.SV();
  const int nv = m.nv, nefc = sv[SV_NEFC];
  real* qacc = c.F(c.L().qacc);
  const bool warm = !(m.opt_disableflags & (1 << 8));
  if (c.lane() == 0) { sv[SV_NITER] = 0; sv[SV_OVF] &= ~(MX_OVERFLOW_ITERATIONS | MX_OVERFLOW_LS_ITERATIONS); }
  for (int i = c.lane(); i < nv; i += kLanes) {
    qacc[i] = (warm && nefc > 0) ? c.F(c.L().warm)[i] : c.F(c.L().qacc_smooth)[i];
    if (nefc == 0) c.F(c.L().qcon)[i] = 0.f;
  }
  sync();
  if (nefc == 0) return;
  islands(c);
#ifdef MX_SLAB
  lint* jmap = c.n() + c.L().cjmap;
  // Workspace route: when this substep's contact Jacobian, column maps, J^T f accumulator and
  // island blocks fit the world's LDS window, the Jacobian is copied there once and the whole
  // solve runs on the LDS copies; else the island blocks alone go to the window if they fit.
  {
    const int ncon = sv[SV_NCON], K = m.maxpairdof, jw = K * ncon;
    const int htotal = c.N(c.L().iblk)[sv[SV_NISL]], hwords = 2 * (htotal + nv + 9 * ncon);
    sdouble* hq = c.hwin() + htotal + nv;                  // contact weights after the blocks and column
    // after the blocks and weights: the Jacobian's values (3 jw words), its column maps (jw), its
    // dof indices (jw 16-bit), J^T f (nv), the contacts' column counts (ncon 16-bit) and the
    // staging vector (nv)
    const int jh = (jw + 1) >> 1, nq = (ncon + 1) >> 1;
    const int base = hwords + 4 * jw + jh + 2 * nv + nq;
    // the rows and contacts: five floats per row, eight per contact, then two 16-bit values per
    // row and three per contact
    const int rows = 6 * nefc + 8 * ncon + ((3 * ncon + 1) >> 1);
    if (base <= c.L().win) {
      sfloat* wf = (sfloat*)c.hwin();
      sfloat* jval = wf + hwords;
      sint* jmap = (sint*)(wf + hwords + 3 * jw);
      sshort* jidx = (sshort*)(wf + hwords + 4 * jw);
      sfloat* qcon = wf + hwords + 4 * jw + jh;
      sshort* qn = (sshort*)(qcon + nv);
      sfloat* xs = qcon + nv + nq;
      const real* gv = c.F(c.L().cjval);
      const int* gi = c.N(c.L().cjidx);
      wave_copy2(jval, gv, 3 * jw, jidx, gi, jw, c.lane());
      if (base + rows <= c.L().win) {
        // the rows and contacts too: every row and contact access of the solve stays in LDS
        WinView wv{jval, jidx, jmap, qcon, c.hwin(), c.hwin() + htotal, hq, qn, xs};
        sfloat* rf = wf + base;
        sshort* ri = (sshort*)(rf + 5 * nefc + 8 * ncon);
        wv.rD = rf; wv.raref = rf + nefc; wv.rjaref = rf + 2 * nefc; wv.rjv = rf + 3 * nefc;
        wv.rforce = rf + 4 * nefc; wv.cdot = rf + 5 * nefc; wv.cfric = rf + 5 * nefc + 3 * ncon;
        wv.rid = ri; wv.rstate = ri + nefc;
        wv.caddr = ri + 2 * nefc; wv.cdim = ri + 2 * nefc + ncon; wv.cjn = ri + 2 * nefc + 2 * ncon;
        wv.copied = true;
        if (nefc <= kLanes && ncon <= kLanes) {
          // one row and one contact per lane: every array's loads issue together, then the stores
          const int l = c.lane();
          int id = 0, adr = 0, dim = 0, cn = 0;
          real rd = 0.f, ra = 0.f, fr[5];
          if (l < nefc) { id = c.N(c.L().rid)[l]; rd = c.F(c.L().rD)[l]; ra = c.F(c.L().raref)[l]; }
          if (l < ncon) { adr = c.N(c.L().caddr)[l]; dim = c.N(c.L().cdim)[l]; cn = c.N(c.L().cjn)[l]; }
#pragma unroll
          for (int k = 0; k < 5; ++k) fr[k] = l + kLanes * k < 5 * ncon ? c.F(c.L().cfric)[l + kLanes * k] : 0.f;
          if (l < nefc) { wv.rid[l] = id; wv.rD[l] = rd; wv.raref[l] = ra; }
          if (l < ncon) { wv.caddr[l] = adr; wv.cdim[l] = dim; wv.cjn[l] = cn; }
#pragma unroll
          for (int k = 0; k < 5; ++k)
            if (l + kLanes * k < 5 * ncon) wv.cfric[l + kLanes * k] = fr[k];
        } else {
          wave_copy(wv.rid, c.N(c.L().rid), nefc, c.lane());
          wave_copy(wv.rD, c.F(c.L().rD), nefc, c.lane());
          wave_copy(wv.raref, c.F(c.L().raref), nefc, c.lane());
          wave_copy(wv.caddr, c.N(c.L().caddr), ncon, c.lane());
          wave_copy(wv.cdim, c.N(c.L().cdim), ncon, c.lane());
          wave_copy(wv.cjn, c.N(c.L().cjn), ncon, c.lane());
          wave_copy(wv.cfric, c.F(c.L().cfric), 5 * ncon, c.lane());
        }
        sync();
        // room left for the saved assembly and the weight changes (incremental Hessian rebuilds)
        const int used = (base + rows + 1) & ~1;
        saved_assembly(c, wv, wf, used, htotal, ncon);
        newton_solve(c, wv);
        return;
      }
      sync();
      WinJView wv{jval, jidx, jmap, qcon, c.hwin(), c.hwin() + htotal, hq, qn, xs};
      working_set_rows(c, wv);
      // room for the saved assembly and the weight changes (incremental Hessian rebuilds)
      const int used = (base + 1) & ~1;
      saved_assembly(c, wv, wf, used, htotal, ncon);
      newton_solve(c, wv);
      return;
    }
    if (hwords <= c.L().win) {   // the island blocks and the contact weights alone
      HWinView hv{c.f() + c.L().cjval, c.n() + c.L().cjidx, jmap, c.f() + c.L().qcon, c.hwin(), c.hwin() + htotal, hq,
                  c.n() + c.L().cqn, nullptr};
      working_set_rows(c, hv);
      newton_solve(c, hv);
      return;
    }
  }
#else
  lint* jmap = nullptr;
#endif
#ifdef MX_SLAB
  WsView ws{c.f() + c.L().cjval, c.n() + c.L().cjidx, jmap, c.f() + c.L().qcon, c.g() + c.L().H, c.g() + c.L().colk,
            c.g() + c.L().cq, c.n() + c.L().cqn, nullptr};
#else
  WsView ws{c.R(c.L().cjval), c.n() + c.L().cjidx, jmap, c.R(c.L().qcon), c.g() + c.L().H, c.g() + c.L().colk,
            nullptr, nullptr, nullptr};
#endif
  working_set_rows(c, ws);
  newton_solve(c, ws);
}

// contacts and rows of the last substep -> HBM (called before that substep's Euler step)
__device__ void publish_constraints(const Ctx& c) {
  KModel& m = c.m();
  KData& d = c.d();
  const int* sv = c.SV();
  size_t w = c.w();
  const int C = m.nconmax, R = m.njmax, ncon = sv[SV_NCON], nefc = sv[SV_NEFC];
  if (c.lane() == 0) { d.ncon[w] = ncon; d.nefc[w] = nefc; d.solver_niter[w] = sv[SV_NITER]; }
  for (int t = c.lane(); t < ncon * 9; t += kLanes) d.contact_frame[9 * C * w + t] = c.F(c.L().cframe)[t];
  for (int t = c.lane(); t < ncon * 5; t += kLanes) d.contact_friction[5 * C * w + t] = c.F(c.L().cfric)[t];
  for (int t = c.lane(); t < ncon * 3; t += kLanes) d.contact_pos[3 * C * w + t] = c.F(c.L().cpos)[t];
  for (int t = c.lane(); t < ncon * 2; t += kLanes) d.contact_geom[2 * C * w + t] = c.N(c.L().cgeom)[t];
  for (int t = c.lane(); t < ncon; t += kLanes) {
    d.contact_dist[C * w + t] = c.F(c.L().cdist)[t];
    d.contact_includemargin[C * w + t] = c.F(c.L().cmargin)[t];
    d.contact_dim[C * w + t] = c.N(c.L().cdim)[t];
  }
  for (int r = c.lane(); r < nefc; r += kLanes) {
    size_t b = (size_t)R * w + r;
    int id = c.N(c.L().rid)[r], type, eid;
    real pos;
    if (id >= 0) {
      int dim = c.N(c.L().cdim)[id];
      type = dim == 1 ? EFC_FRICTIONLESS : (m.opt_cone == 1 ? EFC_ELLIPTIC : EFC_PYRAMIDAL);
      eid = id;
      int comp = r - c.N(c.L().caddr)[id];
      real dist = c.F(c.L().cdist)[id], mg = c.F(c.L().cmargin)[id];
      pos = (m.opt_cone == 1 && comp > 0) ? mg : dist;   // position + margin, position = 0 for cone frictions
    } else {
      real sign;
      int kind;
      int dof = single_dof(id, sign, kind);
      type = kind == 0 ? EFC_FRICTION : EFC_LIMIT;
      eid = kind == 0 ? dof : c.di(dof, D_JNT);
      pos = 0.f;
      if (kind != 0) {
        int j = eid;
        real q = c.F(c.L().qpos)[c.ji(j, J_QPOS)];
        pos = r_min(q - *c.jf(j, J_RANGE), *c.jf(j, J_RANGE + 1) - q);
      }
    }
    d.efc_force[b] = c.F(c.L().rforce)[r];
    d.efc_D[b] = c.F(c.L().rD)[r];
    d.efc_aref[b] = c.F(c.L().raref)[r];
    d.efc_pos[b] = pos;
    d.efc_type[b] = type;
    d.efc_state[b] = c.N(c.L().rstate)[r];
    d.efc_id[b] = eid;
  }
}

template <typename Tv>
__device__ __forceinline__ void put(const Ctx& c, Tv* dst, const real* src, int width) {
  size_t base = (size_t)c.w() * width;
  for (int i = c.lane(); i < width; i += kLanes) dst[base + i] = src[i];
}

// cfrc_ext, cacc, cfrc_int and the force / torque sensors of the last substep, after the
// constraint solve (reference gpu/cuda/dynamics/mjwarp_external_wrench.cu:26-90 initialize_applied /
// accumulate_contacts, mjwarp_postconstraint.cu:87 world_postconstraint, mjwarp_queries.cu:31
// force_torque_sensors); published to HBM.  Spatial quantities are [torque; force] about the
// subtree centre of mass of the body's root.  One lane per body sums its contacts in contact order
// (deterministic, no atomics); this runs once per launch.
template <bool kRows>
__device__ void post_constraint(const Ctx& c) {
  KModel& m = c.m();
  KData& d = c.d();
  const size_t w = c.w();
  real* ext = c.F(c.L().cext);
  const real* x = c.F(c.L().xfrc);
  const bool xf = c.MISC()[kXfrc] != 0;
  const real* scom = c.F(c.L().scom);
  for (int b = c.lane(); b < m.nbody; b += kLanes) {
    real w6[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (xf) point_wrench(c, b, x + 6 * b, x + 6 * b + 3, w6);
    if (kRows && b > 0) {
      const int ncon = c.SV()[SV_NCON];
      const real* sc = scom + 3 * c.bi(b, B_ROOT);
      for (int con = 0; con < ncon; ++con) {
        const int b1 = c.gi(c.N(c.L().cgeom)[2 * con], G_BODY), b2 = c.gi(c.N(c.L().cgeom)[2 * con + 1], G_BODY);
        const int adr = c.N(c.L().caddr)[con];
        if ((b1 != b && b2 != b) || adr < 0) continue;
        const int dim = c.N(c.L().cdim)[con];
        const real* f = c.F(c.L().rforce) + adr;
        const real* mu = c.F(c.L().cfric) + 5 * con;
        real l0 = 0.f, l1 = 0.f, l2 = 0.f;
        if (dim == 1) {
          l0 = f[0];
        } else if (m.opt_cone == 0) {   // pyramidal edges (n + mu t, n - mu t) per tangent
          l0 = f[0] + f[1] + f[2] + f[3];
          l1 = (f[0] - f[1]) * mu[0];
          l2 = (f[2] - f[3]) * mu[1];
        } else {
          l0 = f[0]; l1 = f[1]; l2 = f[2];
        }
        const real* fr = c.F(c.L().cframe) + 9 * con;   // rows: normal, tangent 1, tangent 2
        const real F[3] = {fr[0] * l0 + fr[3] * l1 + fr[6] * l2, fr[1] * l0 + fr[4] * l1 + fr[7] * l2,
                            fr[2] * l0 + fr[5] * l1 + fr[8] * l2};
        const real* p = c.F(c.L().cpos) + 3 * con;
        const real off[3] = {p[0] - sc[0], p[1] - sc[1], p[2] - sc[2]};
        real t[3];
        cross3(off, F, t);
        const real sign = b == b2 ? 1.f : -1.f;
        for (int k = 0; k < 3; ++k) { w6[k] += sign * t[k]; w6[3 + k] += sign * F[k]; }
      }
    }
    for (int k = 0; k < 6; ++k) ext[6 * b + k] = w6[k];
  }
  sync();
  // accelerations with the solved qacc, then the bodies' net forces minus the external ones
  const real* qvel = c.F(c.L().qvel);
  const real* qacc = c.F(c.L().qacc);
  real* cacc = c.F(c.L().cacc);
  real* cfb = c.F(c.L().cfrcb);
  const real* ci = c.F(c.L().cinert);
  const real* cvel = c.F(c.L().cvel);
  real g[3] = {0.f, 0.f, 0.f};
  if (!(m.opt_disableflags & (1 << 6))) { g[0] = -m.opt_gravity_x; g[1] = -m.opt_gravity_y; g[2] = -m.opt_gravity_z; }
  for (int b = c.lane(); b < m.nbody; b += kLanes) {
    real a[6] = {0.f, 0.f, 0.f, g[0], g[1], g[2]};
    if (b > 0) {
      chain_axpy(c.chain(b), c.F(c.L().cdofdot), qvel, a);
      chain_axpy(c.chain(b), c.F(c.L().cdof), qacc, a);
    }
    for (int k = 0; k < 6; ++k) cacc[6 * b + k] = a[k];
    if (b == 0) { for (int k = 0; k < 6; ++k) cfb[k] = 0.f; continue; }
    real f1[6], h[6], f2[6];
    mul_inert_vec(ci + 10 * b, a, f1);
    mul_inert_vec(ci + 10 * b, cvel + 6 * b, h);
    cross_force(cvel + 6 * b, h, f2);
    for (int k = 0; k < 6; ++k) cfb[6 * b + k] = f1[k] + f2[k] - ext[6 * b + k];
  }
  sync();
  real* cint = c.F(c.L().cfrc);
  for (int t = c.lane(); t < 6 * m.nbody; t += kLanes) {
    int b = t / 6, k = t % 6;
    cint[t] = b > 0 ? range_sum(cfb + k, 6, b, b + c.bi(b, B_SUBTREE)) : 0.f;
  }
  sync();
  for (int s = c.lane(); s < m.nsensor; s += kLanes) {
    const int site = m.sensor_objid[s], b = c.si(site, S_BODY);
    const real* wr = cint + 6 * b;
    real v[3];
    if (m.sensor_type[s] == MX_SENS_FORCE) {
      for (int k = 0; k < 3; ++k) v[k] = wr[3 + k];
    } else {
      const real* sc = scom + 3 * c.bi(b, B_ROOT);
      const real* sp = c.F(c.L().sxpos) + 3 * site;
      const real off[3] = {sp[0] - sc[0], sp[1] - sc[1], sp[2] - sc[2]}, fv[3] = {wr[3], wr[4], wr[5]};
      real t[3];
      cross3(off, fv, t);
      for (int k = 0; k < 3; ++k) v[k] = wr[k] - t[k];
    }
    const real* R = c.F(c.L().sxmat) + 9 * site;
    const real cut = m.sensor_cutoff[s];
    const int type = m.sensor_datatype[s], adr = m.sensor_adr[s];
    for (int k = 0; k < 3; ++k) {
      real o = R[k] * v[0] + R[3 + k] * v[1] + R[6 + k] * v[2];   // site frame
      if (cut > 0.f) {
        if (type == 0) o = r_min(cut, r_max(-cut, o));
        else if (type == 1) o = r_min(cut, o);
      }
      d.sensordata[w * m.nsensordata + adr + k] = o;
    }
  }
  put(c, d.cacc, cacc, 6 * m.nbody);
  put(c, d.cfrc_int, cint, 6 * m.nbody);
  put(c, d.cfrc_ext, ext, 6 * m.nbody);
}

// ---------------------------------------------------------------- kernel
__device__ void load_world(const Ctx& c) {
  KModel& m = c.m();
  KData& d = c.d();
  size_t w = c.w();
#ifndef MX_SLAB
  stage_image(m, c.I(), (float*)c.fi(), c.lane(), kLanes);   // the workspace route stages it once per launch
#endif
  for (int i = c.lane(); i < m.nq; i += kLanes) c.F(c.L().qpos)[i] = d.qpos[w * m.nq + i];
  for (int i = c.lane(); i < m.nv; i += kLanes) {
    c.F(c.L().qvel)[i] = d.qvel[w * m.nv + i];
    c.F(c.L().warm)[i] = d.qacc_warmstart[w * m.nv + i];
    c.F(c.L().applied)[i] = d.qfrc_applied[w * m.nv + i];
  }
  for (int i = c.lane(); i < m.nu; i += kLanes) c.F(c.L().ctrl)[i] = d.ctrl[w * m.nu + i];
  bool xfrc = false;   // applied body wrenches: any nonzero entry switches their projection on
  for (int i = c.lane(); i < 6 * m.nbody; i += kLanes) {
    const real v = d.xfrc_applied[w * 6 * m.nbody + i];
    c.F(c.L().xfrc)[i] = v;
    xfrc |= v != 0.f;
  }
  xfrc = __any(xfrc);
  if (c.lane() < 3) c.D(c.L().goalpos)[c.lane()] = d.osc_goal_pos[3 * w + c.lane()];
  if (c.lane() < 9) c.D(c.L().goalrot)[c.lane()] = d.osc_goal_rot[9 * w + c.lane()];
  if (c.lane() < 2) c.D(c.L().grip)[c.lane()] = d.osc_gripper[2 * w + c.lane()];
  // the pose delta scaled once per launch; the gripper command as given
  if (c.lane() < 7)
    c.D(c.L().action)[c.lane()] = c.lane() < 6 ? scaled_action(m, d, w, c.lane()) : d.osc_action[7 * w + 6];
  if (c.lane() < 12) c.D(c.L().gains)[c.lane()] = d.osc_gains[12 * w + c.lane()];
  if (c.lane() < m.osc_ndof) c.D(c.L().q0)[c.lane()] = d.osc_q0[m.osc_ndof * w + c.lane()];
  if (c.lane() < m.osc_ndof) c.D(c.L().tau)[c.lane()] = d.osc_tau[m.osc_ndof * w + c.lane()];
  if (m.has_body_active && m.njmax > 0)
    for (int i = c.lane(); i < m.nbody; i += kLanes) c.N(c.L().bact)[i] = d.body_active[w * m.nbody + i];
  int* misc = c.MISC();
  if (c.lane() < 16) misc[c.lane()] = 0;
  if (c.lane() < 32) c.SV()[c.lane()] = 0;
  sync();
  if (c.lane() == 0) {
    misc[kCtrlErr] = d.osc_error[w];
    misc[kMaxTree] = m.maxtree;
    misc[kXfrc] = xfrc;
    for (int k = 0; k < 3; ++k) misc[kRank0 + k] = d.osc_rank[3 * w + k];
  }
  sync();
}

__device__ void publish_derived(const Ctx& c) {
  KModel& m = c.m();
  KData& d = c.d();
  int nv = m.nv, nb = m.nbody;
  put(c, d.qacc, c.F(c.L().qacc), nv);
  put(c, d.qacc_smooth, c.F(c.L().qacc_smooth), nv);
  put(c, d.qfrc_bias, c.F(c.L().bias), nv);
  put(c, d.qfrc_passive, c.F(c.L().passive), nv);
  put(c, d.qfrc_actuator, c.F(c.L().act), nv);
  put(c, d.qfrc_smooth, c.F(c.L().smooth), nv);
  put(c, d.qfrc_constraint, c.F(c.L().qcon), nv);
  put(c, d.actuator_force, c.F(c.L().actforce), m.nu);
  put(c, d.M, c.F(c.L().M), m.nM);
  put(c, d.xpos, c.F(c.L().xpos), 3 * nb);
  put(c, d.xquat, c.F(c.L().xquat), 4 * nb);
  put(c, d.xmat, c.F(c.L().xmat), 9 * nb);
  put(c, d.geom_xpos, c.F(c.L().gxpos), 3 * m.ngeom);
  put(c, d.geom_xmat, c.F(c.L().gxmat), 9 * m.ngeom);
  put(c, d.site_xpos, c.F(c.L().sxpos), 3 * m.nsite);
  put(c, d.site_xmat, c.F(c.L().sxmat), 9 * m.nsite);
  put(c, d.subtree_com, c.F(c.L().scom), 3 * nb);
}

__device__ void store_world(const Ctx& c, int integrated) {
  KModel& m = c.m();
  KData& d = c.d();
  size_t w = c.w();
  put(c, d.qpos, c.F(c.L().qpos), m.nq);
  put(c, d.qvel, c.F(c.L().qvel), m.nv);
  put(c, d.qacc_warmstart, c.F(c.L().warm), m.nv);
  put(c, d.ctrl, c.F(c.L().ctrl), m.nu);
  int* misc = c.MISC();
  if (c.lane() < 3) d.osc_goal_pos[3 * w + c.lane()] = c.D(c.L().goalpos)[c.lane()];
  if (c.lane() < 9) d.osc_goal_rot[9 * w + c.lane()] = c.D(c.L().goalrot)[c.lane()];
  if (c.lane() < 2) d.osc_gripper[2 * w + c.lane()] = c.D(c.L().grip)[c.lane()];
  if (c.lane() < m.osc_ndof) d.osc_tau[m.osc_ndof * w + c.lane()] = c.D(c.L().tau)[c.lane()];
  if (c.lane() < 3) d.osc_rank[3 * w + c.lane()] = misc[kRank0 + c.lane()];
  if (c.lane() == 0) {
    d.osc_error[w] = misc[kCtrlErr];
    // capacity and failure bits stay set until the caller clears them (a reset); the solver's
    // iteration-limit bits describe the last substep only
    constexpr int kLast = MX_OVERFLOW_ITERATIONS | MX_OVERFLOW_LS_ITERATIONS;
    d.overflow[w] = (d.overflow[w] & ~kLast) | c.SV()[SV_OVF];
    d.nstep[w] += integrated;
    d.time[w] += integrated * m.opt_timestep;
    if (m.njmax > 0)   // sticky like nstep: the caller clears them
      for (int k = 0; k < 4; ++k) d.stat_sums[4 * w + k] += (double)c.SV()[SV_STAT + k];
  }
}

// kRows: the model has constraint rows (contacts, limits, dof friction).  The smooth-only
// instantiation carries none of the collision / Newton code, so its register allocation is that
// of the smooth stages alone.
// Minimum waves per SIMD the register allocation must allow.  In LDS the contact kernel holds
// 60-125 KB per world, so at most two worlds share a CU and registers are not the limit.  With the
// working set in workspace slabs the only limit is registers: four waves per SIMD (128 VGPRs)
// hides the slabs' memory latency best (measured 1 to 8 waves per SIMD: 4 is fastest on C3, C4,
// C5; fewer registers spill more).
#ifdef MX_SLAB
constexpr int kMinWaves(bool rows) { return rows ? 4 : 2; }
#else
constexpr int kMinWaves(bool rows) { return rows ? 1 : 2; }
#endif

// The observation plan sampled by the world's wave after a substep: qpos and qvel after the
// substep's integration, body and site poses before it.
__device__ __forceinline__ void sample_plan(const Ctx& c) {
  KParams& p = params();
  KModel& m = p.m;
  KLayout& L = p.L;
  const real* qp = c.F(L.qpos);
  const real* qv = c.F(L.qvel);
  const real* sx = c.F(L.sxpos);
  const real* bx = c.F(L.xpos);
  const real* bq = c.F(L.xquat);
  const int nq = m.nq, nv = m.nv, ns3 = 3 * m.nsite, nb3 = 3 * m.nbody, nb4 = 4 * m.nbody;
  obs_sample(p.obs, (size_t)c.w(), c.lane(), m.opt_timestep, 0, [&](int code) -> float {
    const int e = code & 0xffffff;
    switch (code >> 24) {
      case MX_OBS_SRC_QPOS: return e < nq ? qp[e] : 0.f;
      case MX_OBS_SRC_QVEL: return e < nv ? qv[e] : 0.f;
      case MX_OBS_SRC_SITE_XPOS: return e < ns3 ? sx[e] : 0.f;
      case MX_OBS_SRC_XPOS: return e < nb3 ? bx[e] : 0.f;
      case MX_OBS_SRC_XQUAT: return e < nb4 ? bq[e] : 0.f;
      default: return 0.f;
    }
  });
  sync();
}

#ifdef MX_SLAB
// Substep starts of the current launch, summed over the worlds of each of eight groups (world index
// mod 8, which is how workgroups spread over the eight XCDs), one counter per 256 bytes so that the
// groups' atomics do not queue on one address; zeroed by image_kernel, which runs before every
// workspace-route launch on the same stream.  control_step_kernel paces its worlds by them
// (launches that overlap on one device share the counters, which skews their priorities only).
constexpr int kPaceGroups = 8, kPaceStride = 64;
__device__ __align__(256) unsigned int g_substeps_started[kPaceGroups * kPaceStride];
#endif

template <bool kRows>
// The parameter block is read through params() (the kernel argument segment), never through the
// by-value parameter, so no private copy of it is made.
__global__ __launch_bounds__(kLanes, kMinWaves(kRows)) void control_step_kernel(Params) {
  {
    // params() addresses the block back from the hidden arguments; a compiler that placed them
    // elsewhere would make every read wrong, so the kernel checks the placement first (in its own
    // body the segment pointer is valid) and flags the world instead of computing.
    typedef const __attribute__((address_space(4))) unsigned char KByte;
    KByte* seg = (KByte*)__builtin_amdgcn_kernarg_segment_ptr();
    if (seg + sizeof(Params) != (KByte*)__builtin_amdgcn_implicitarg_ptr()) {
      KParams& kp = *(KParams*)seg;
      if (threadIdx.x == 0 && (int)blockIdx.x < kp.d.nworld) kp.d.overflow[blockIdx.x] |= MX_OVERFLOW_LAUNCH;
      return;
    }
  }
  KParams& p = params();
  KModel& m = p.m;
  KLayout& L = p.L;
  const int substeps = p.substeps, flags = p.flags;
  const int w = blockIdx.x;
  if (w >= p.d.nworld) return;
  if (p.mask && !p.mask[w]) return;
  const Ctx c;
  load_world(c);
  bool damped = false;
  if (!(m.opt_disableflags & (1 << 15)))
    for (int i = 0; i < m.nv; ++i) damped |= c.df(i, D_DAMP) > 0.f;
  int integrated = 0;
#ifdef MX_SLAB
  // A launch lasts as long as its slowest world, and the worlds of one CU share its SIMDs: a world
  // whose substeps trail its group's mean by more than one and a half raises its wave's issue
  // priority until it catches up.  Each substep start adds one to the group's counter (a relaxed
  // atomic whose old value the next substep reads); this changes scheduling only, never results.
  // Only launches whose worlds are all resident at once are paced (the mean then means progress).
  unsigned int started = 0;   // lane 0: the group's substep starts before this world's last one
  // the worlds of this world's group (w mod 8), and its counter
  const unsigned int nw = (unsigned int)((p.d.nworld - (w & (kPaceGroups - 1)) + kPaceGroups - 1) / kPaceGroups);
  unsigned int* pace_ctr = g_substeps_started + (w & (kPaceGroups - 1)) * kPaceStride;
  const bool pace = kRows && p.pace;
#endif
  for (int s = 0; s < substeps; ++s) {
    const int policy = (flags & MX_FLAG_POLICY_FIRST) && s == 0;
#ifdef MX_SLAB
    if (pace) {
      // at this world's start of substep s - 1 the group's worlds had started before / nw
      // substeps on average, against this world's s - 1: behind by more than 1.5 substeps
      const unsigned int before = __builtin_amdgcn_readfirstlane(started);
      if (s > 0 && 2ull * before > (2ull * s + 1ull) * nw) __builtin_amdgcn_s_setprio(2);
      else __builtin_amdgcn_s_setprio(0);
      if (threadIdx.x == 0) started = __hip_atomic_fetch_add(pace_ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#endif
    kinematics(c);
    com_pos(c);
    crb_mass(c);
    mass_inverse(c, c.R(L.M), c.R(L.Minv), damped, m.opt_timestep);
    if (kRows) {
      collide(c);
      make_rows(c);
    }
    velocity(c);
    if ((flags & MX_FLAG_BOOTSTRAP) && s == 0) {
      const real* sp = c.F(L.sxpos) + 3 * m.osc_site;
      const real* sr = c.F(L.sxmat) + 9 * m.osc_site;
      if (c.lane() < 3) c.D(L.goalpos)[c.lane()] = sp[c.lane()];
      if (c.lane() < 9) c.D(L.goalrot)[c.lane()] = sr[c.lane()];
      if (c.lane() < 2) c.D(L.grip)[c.lane()] = 0.0;
      if (c.lane() == 0) c.MISC()[kCtrlErr] = 0;
      sync();
    }
    if (!(flags & MX_FLAG_NO_CONTROL)) control<false>(c, policy, s == substeps - 1 || (flags & MX_FLAG_NO_INTEGRATE));
    actuation(c);
    if (kRows) {
      newton(c);
      if (c.lane() == 0) {   // the substep's rows, contacts and Newton iterations, summed over the launch
        int* sv = c.SV();
        sv[SV_STAT] += sv[SV_NEFC];
        sv[SV_STAT + 1] += sv[SV_NCON];
        sv[SV_STAT + 2] += sv[SV_NITER];
        sv[SV_STAT + 3] += sv[SV_NITER] * sv[SV_NEFC];
      }
    } else {
      for (int i = c.lane(); i < m.nv; i += kLanes) {
        c.F(L.qacc)[i] = c.F(L.qacc_smooth)[i];
        c.F(L.qcon)[i] = 0.f;
      }
      sync();
    }
    // the last substep's contacts and rows, published before Euler moves qpos (a limit row's
    // efc_pos is its distance at build time, as the reference's row_pos)
    const bool last = (flags & MX_FLAG_NO_INTEGRATE) || s == substeps - 1;
    if (last) {
      post_constraint<kRows>(c);
      if (kRows) publish_constraints(c);
      sync();
    }
    if (flags & MX_FLAG_NO_INTEGRATE) break;
    euler(c, damped);
    ++integrated;
    // the observation plan: qpos and qvel after this substep's integration, poses before it
    if (p.obs.nspec > 0) sample_plan(c);
  }
  // derived fields of the last substep are still in LDS (Euler writes only qpos, qvel, warmstart)
  publish_derived(c);
  store_world(c, integrated);
}

#ifndef MX_SLAB
// The smooth path (models without constraint rows, LDS route) with two wavefronts per world, for
// batches that leave most wave slots free: wave 0 runs the position stages, then the velocity stage
// and the mass-matrix inverses while wave 1 runs the FP64 controller up to its bias-free torque
// terms (control(), which needs the positions and M only); wave 0 then adds the bias force
// (control_bias()) and runs actuation, the post-constraint stage, Euler and the observation
// sampling.  Between two of this kernel's workgroup barriers the waves write disjoint parts of the
// working set (velocity, bias, passive forces, the inverses and their Gauss-Jordan buffers; the
// controller's Jacobians, its FP64 temporaries in the LDS window, goal and gripper), and both reach
// the barriers in the same order, the flags and substep count being uniform.  The results are
// those of control_step_kernel<false>.
__global__ __launch_bounds__(2 * kLanes, 2) void control_step_kernel_smooth(Params) {
  {
    typedef const __attribute__((address_space(4))) unsigned char KByte;
    KByte* seg = (KByte*)__builtin_amdgcn_kernarg_segment_ptr();
    if (seg + sizeof(Params) != (KByte*)__builtin_amdgcn_implicitarg_ptr()) {
      KParams& kp = *(KParams*)seg;
      if (threadIdx.x == 0 && (int)blockIdx.x < kp.d.nworld) kp.d.overflow[blockIdx.x] |= MX_OVERFLOW_LAUNCH;
      return;
    }
  }
  KParams& p = params();
  KModel& m = p.m;
  KLayout& L = p.L;
  const int substeps = p.substeps, flags = p.flags;
  const int w = blockIdx.x;
  if (w >= p.d.nworld) return;
  if (p.mask && !p.mask[w]) return;
  const int wave = (int)threadIdx.x / kLanes;
  const Ctx c;
  if (wave == 0) load_world(c);
  __syncthreads();
  bool damped = false;
  if (!(m.opt_disableflags & (1 << 15)))
    for (int i = 0; i < m.nv; ++i) damped |= c.df(i, D_DAMP) > 0.f;
  int integrated = 0;
  for (int s = 0; s < substeps; ++s) {
    const int policy = (flags & MX_FLAG_POLICY_FIRST) && s == 0;
    const bool last = (flags & MX_FLAG_NO_INTEGRATE) || s == substeps - 1;
    if (wave == 0) {
      kinematics(c);
      com_pos(c);
      crb_mass(c);
    }
    __syncthreads();
    if (wave == 0) {
      velocity(c);
      mass_inverse(c, c.R(L.M), c.R(L.Minv), damped, m.opt_timestep);
    } else {
      if ((flags & MX_FLAG_BOOTSTRAP) && s == 0) {
        const real* sp = c.F(L.sxpos) + 3 * m.osc_site;
        const real* sr = c.F(L.sxmat) + 9 * m.osc_site;
        if (c.lane() < 3) c.D(L.goalpos)[c.lane()] = sp[c.lane()];
        if (c.lane() < 9) c.D(L.goalrot)[c.lane()] = sr[c.lane()];
        if (c.lane() < 2) c.D(L.grip)[c.lane()] = 0.0;
        if (c.lane() == 0) c.MISC()[kCtrlErr] = 0;
        sync();
      }
      if (!(flags & MX_FLAG_NO_CONTROL)) control<true>(c, policy, last);
    }
    __syncthreads();
    if (wave == 0) {
      if (!(flags & MX_FLAG_NO_CONTROL)) control_bias(c, last);
      actuation(c);
      for (int i = c.lane(); i < m.nv; i += kLanes) {
        c.F(L.qacc)[i] = c.F(L.qacc_smooth)[i];
        c.F(L.qcon)[i] = 0.f;
      }
      sync();
      if (last) {
        post_constraint<false>(c);
        sync();
      }
      if (!(flags & MX_FLAG_NO_INTEGRATE)) {
        euler(c, damped);
        if (p.obs.nspec > 0) sample_plan(c);
      }
    }
    if (flags & MX_FLAG_NO_INTEGRATE) break;
    ++integrated;
  }
  if (wave == 0) {
    publish_derived(c);
    store_world(c, integrated);
  }
}
#endif

const char* kFieldTables[7][64] = {
#define NM(name) #name,
    {MX_MODEL_REAL_ARRAYS(NM)}, {MX_MODEL_INT_ARRAYS(NM)}, {MX_MODEL_INT_SCALARS(NM)},
    {MX_MODEL_REAL_SCALARS(NM)}, {MX_DATA_REAL_ARRAYS(NM)}, {MX_DATA_F64_ARRAYS(NM)}, {MX_DATA_INT_ARRAYS(NM)}
#undef NM
};

int count_names(int which) {
  int n = 0;
  while (n < 64 && kFieldTables[which][n]) ++n;
  return n;
}

// Bytes of one world's slab in the workspace (a multiple of 256, so every slab stays aligned).
size_t slab_bytes(const Layout& L) { return ((size_t)L.bytes + 255) / 256 * 256; }

// Launch the step kernel of this build (LDS working set, or workspace slabs when MX_SLAB is set).
#ifdef MX_SLAB
// Workspace route: one workgroup writes the model image into slab 0, where every world of the
// launch reads it (one copy in the caches instead of one per world).
__global__ __launch_bounds__(256) void image_kernel(Params) {
  {   // the placement check of control_step_kernel (which flags the worlds)
    typedef const __attribute__((address_space(4))) unsigned char KByte;
    if ((KByte*)__builtin_amdgcn_kernarg_segment_ptr() + sizeof(Params) != (KByte*)__builtin_amdgcn_implicitarg_ptr())
      return;
  }
  KParams& p = params();
  if (threadIdx.x < kPaceGroups) g_substeps_started[threadIdx.x * kPaceStride] = 0u;
  stage_image(p.m, p.I, reinterpret_cast<float*>(p.d.workspace) + p.L.img, (int)threadIdx.x, (int)blockDim.x);
}
#endif

#ifdef MX_SLAB
// Whether a launch's worlds are all resident at once: each CU holds 4 waves per SIMD (the kernel's
// register budget) or fewer when their LDS windows fill its 160 KB.
static bool all_resident(int nworld, size_t shared) {
  static int ncu[64];   // per device, filled on first use (a benign race: every writer stores the same)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  if (ncu[dev] <= 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return false;
    ncu[dev] = v;
  }
  const long long by_lds = 163840 / (long long)shared, per_cu = by_lds < 4 * kMinWaves(true) ? by_lds : 4 * kMinWaves(true);
  return (long long)nworld <= (long long)ncu[dev] * per_cu;
}
#endif

int launch_kernel(const MxModel* m, const MxData* d, const int32_t* mask, int substeps, int flags, void* stream,
                  const MxObsPlan* obs) {
  MxObsPlan none{};
  Params p{*m, *d, make_layout(*m), image_layout(*m), substeps, flags, mask, obs ? *obs : none, 0};
#ifdef MX_SLAB
  const size_t shared = (p.L.win + kLdsScalars) * sizeof(float);   // the LDS window, then misc and sv
  p.pace = all_resident(d->nworld, shared) ? 1 : 0;
  hipLaunchKernelGGL(image_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, p);
#else
  const size_t shared = p.L.bytes;
#endif
  if (m->njmax > 0)
    hipLaunchKernelGGL(control_step_kernel<true>, dim3(d->nworld), dim3(kLanes), shared, (hipStream_t)stream, p);
  else
#ifdef MX_SLAB
    hipLaunchKernelGGL(control_step_kernel<false>, dim3(d->nworld), dim3(kLanes), shared, (hipStream_t)stream, p);
#else
    hipLaunchKernelGGL(control_step_kernel_smooth, dim3(d->nworld), dim3(2 * kLanes), shared, (hipStream_t)stream, p);
#endif
  return (int)hipGetLastError();
}

#ifdef MX_F64
int lds_bytes_for(const MxModel* m) { return make_layout(*m).bytes; }
#endif

#ifndef MX_SLAB
int device_lds_limit() {
  int dev = 0, value = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 65536;
  if (hipDeviceGetAttribute(&value, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) return 65536;
  return value;
}

#endif

}  // namespace MX_NS

#if !defined(MX_SLAB) && !defined(MX_F64)
namespace mx_slab {
size_t slab_bytes_for(const MxModel* m);
int launch_kernel(const MxModel* m, const MxData* d, const int32_t* mask, int substeps, int flags, void* stream,
                  const MxObsPlan* obs);
}  // namespace mx_slab
namespace mx_slab4 {
int launch_kernel(const MxModel* m, const MxData* d, const int32_t* mask, int substeps, int flags, void* stream,
                  const MxObsPlan* obs);
}  // namespace mx_slab4
namespace mx_f64 {
int lds_bytes_for(const MxModel* m);
int launch_kernel(const MxModel* m, const MxData* d, const int32_t* mask, int substeps, int flags, void* stream,
                  const MxObsPlan* obs);
}  // namespace mx_f64

namespace mx {
// A usable workspace: 256-byte slabs of at least mx_workspace_bytes, one per world plus slab 0.
bool workspace_ok(const MxModel* m, const MxData* d) {
  return d->workspace && d->workspace_doubles > 0 && d->workspace_doubles % 32 == 0 &&
         (size_t)d->workspace_doubles * 8 >= mx_slab::slab_bytes_for(m) &&
         d->workspace_total >= (int64_t)(d->nworld + 1) * d->workspace_doubles;
}

int launch(const MxModel* m, const MxData* d, const int32_t* mask, int substeps, int flags, void* stream,
           const MxObsPlan* obs = nullptr) {
  int rc = mx_check(m, d);
  if (rc) return rc;
  if (substeps < 1) return MX_ERR_INVALID;
  if (flags & MX_FLAG_FP64) {   // the FP64 route: its working set in LDS, or nothing
    const int bytes = mx_f64::lds_bytes_for(m);
    if (bytes > MX_LDS_BUDGET || bytes > device_lds_limit()) return MX_ERR_LDS;
    return mx_f64::launch_kernel(m, d, mask, substeps, flags, stream, obs);
  }
  Layout L = make_layout(*m);
  const bool fits = L.bytes <= MX_LDS_BUDGET && L.bytes <= device_lds_limit();
  const bool have = workspace_ok(m, d);
  // route: workspace slabs when forced, when the working set exceeds LDS, or by default for models
  // with constraint rows when a workspace is given (higher occupancy); LDS otherwise
  bool slab = (flags & MX_FLAG_WORKSPACE) || !fits || (m->njmax > 0 && have);
  if ((flags & MX_FLAG_LDS) && fits) slab = false;
  if (!slab) return launch_kernel(m, d, mask, substeps, flags, stream, obs);
  if (!have) return MX_ERR_LDS;
  // contact-free island blocks: sum over trees of n (n + 1) / 2 = (nM + nv) / 2 packed entries
  if ((m->nM + m->nv) / 2 <= 192) return mx_slab4::launch_kernel(m, d, mask, substeps, flags, stream, obs);
  return mx_slab::launch_kernel(m, d, mask, substeps, flags, stream, obs);
}

// ---- fixed device scratch of mx_control_step_noalloc
// The workspace slabs of callers that cannot allocate device memory: one array per device,
// reserved with the code object and held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol): each device's
// address comes from hipGetSymbolAddress, taken once per device with that device current.
constexpr size_t kScratchDoubles = MX_SCRATCH_BYTES / sizeof(double);
static __device__ __align__(256) double scratch[kScratchDoubles];

constexpr int kMaxDevices = 64;
double* g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

// This device's copy of `scratch` (the current device's, resolved on its first successful use).
// Only a resolved address is kept: a failed hipGetSymbolAddress returns its error and the next call
// tries again, so a transient failure (for instance a first call made while another thread's stream
// capture forbids the runtime's lazy code-object load) does not disable the entry for the process.
int scratch_of_current_device(double** out) {
  int dev = 0;
  hipError_t rc = hipGetDevice(&dev);
  if (rc != hipSuccess) return (int)rc;
  if (dev < 0 || dev >= kMaxDevices) return MX_ERR_INVALID;
  std::lock_guard<std::mutex> hold(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (rc != hipSuccess) return (int)rc;
    if (!p) return MX_ERR_INVALID;
    g_scratch_ptr[dev] = static_cast<double*>(p);
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

int control_step_noalloc(const MxModel* m, const MxData* d, int substeps, int flags, void* stream) {
  if (!m || !d || d->nworld < 1) return MX_ERR_INVALID;
  MxData local = *d;
  local.workspace = nullptr;
  local.workspace_doubles = 0;
  local.workspace_total = 0;
  // the workspace route runs models with constraint rows and models beyond the LDS budget
  if (m->njmax > 0 || make_layout(*m).bytes > MX_LDS_BUDGET) {
    const size_t slab = mx_slab::slab_bytes_for(m) / sizeof(double);   // a multiple of 32 doubles
    if ((size_t)(d->nworld + 1) * slab > kScratchDoubles) return MX_ERR_SCRATCH;
    double* ptr = nullptr;
    const int rc = scratch_of_current_device(&ptr);
    if (rc) return rc;
    local.workspace = ptr;
    local.workspace_doubles = (int32_t)slab;
    local.workspace_total = (int64_t)kScratchDoubles;
  }
  return launch(m, &local, nullptr, substeps, flags & ~MX_FLAG_NO_INTEGRATE, stream);
}

// ---- the FP64 OSC alone (mx_osc): the controller of every world from its published inputs
struct OscParams {
  MxModel m;
  MxData d;
  Layout L;
  int flags;
};
typedef const __attribute__((address_space(4))) OscParams KOscParams;

// The standalone controller's world context for control_solve(): the controller's doubles (state
// and temporaries at the layout's double offsets) and its scalar slots in LDS, the model read in
// place in the kernel argument segment.
struct OscCtx {
  KOscParams* p;
  double* dbl;
  int* misc;
  __device__ KModel& m() const { return p->m; }
  __device__ KLayout& L() const { return p->L; }
  __device__ int lane() const { return (int)threadIdx.x; }
  __device__ int* MISC() const { return misc; }
  __device__ double* O(int off) const { return dbl + off; }
  __device__ double* D(int off) const { return dbl + off; }
  __device__ int osc_act(int i) const { return p->m.osc_actuator[i]; }
  __device__ real ctrlrange(int a, int k) const { return p->m.actuator_ctrlrange[2 * a + k]; }
};

// One wavefront per world (the reference's standalone controller kernel, control / control_fast,
// gpu/cuda/control/osc_solver.cu:309-727, over ControllerSolveData): the inputs are the world's
// published osc_mass, osc_jac, osc_q, osc_qvel, osc_bias and end-effector pose and velocity; the
// outputs osc_tau, ctrl of the OSC actuators, the goal (policy step), gripper, error and ranks.
__global__ __launch_bounds__(kLanes) void osc_kernel(OscParams) {
  KOscParams* kp = (KOscParams*)__builtin_amdgcn_kernarg_segment_ptr();
  const int w = blockIdx.x, lane = threadIdx.x;
  if (w >= kp->d.nworld) return;
  KData& d = kp->d;
  KLayout& L = kp->L;
  const size_t ww = (size_t)w;
  const int nu = kp->m.nu;
  double* dbl = (double*)mx_lds;
  int* misc = (int*)(dbl + L.otmp_end);
  float* ctrl = (float*)(misc + 16);
  const OscCtx c{kp, dbl, misc};
  if (lane < 3) dbl[L.goalpos + lane] = d.osc_goal_pos[3 * ww + lane];
  if (lane < 9) dbl[L.goalrot + lane] = d.osc_goal_rot[9 * ww + lane];
  if (lane < 2) dbl[L.grip + lane] = d.osc_gripper[2 * ww + lane];
  const int on = kp->m.osc_ndof;
  if (lane < 7) dbl[L.action + lane] = lane < 6 ? scaled_action(kp->m, d, ww, lane) : d.osc_action[7 * ww + 6];
  if (lane < on) {
    dbl[L.q0 + lane] = d.osc_q0[on * ww + lane];
    dbl[L.tau + lane] = d.osc_tau[on * ww + lane];
    dbl[L.q + lane] = d.osc_q[on * ww + lane];
    dbl[L.qd + lane] = d.osc_qvel[on * ww + lane];
    dbl[L.dbias + lane] = d.osc_bias[on * ww + lane];
  }
  if (lane < 12) dbl[L.gains + lane] = d.osc_gains[12 * ww + lane];
  if (lane < on * on) dbl[L.m7 + lane] = d.osc_mass[on * on * ww + lane];
  if (lane < 6 * on) dbl[L.J + lane] = d.osc_jac[6 * on * ww + lane];
  if (lane < 3) dbl[L.eepos + lane] = d.osc_ee_pos[3 * ww + lane];
  if (lane < 9) dbl[L.eerot + lane] = d.osc_ee_rot[9 * ww + lane];
  if (lane < 6) dbl[L.eevel + lane] = d.osc_ee_vel[6 * ww + lane];
  for (int a = lane; a < nu; a += kLanes) ctrl[a] = d.ctrl[ww * nu + a];
  if (lane < 16) misc[lane] = 0;
  sync();
  if (lane == 0) {
    misc[kCtrlErr] = d.osc_error[ww];
    for (int k = 0; k < 3; ++k) misc[kRank0 + k] = d.osc_rank[3 * ww + k];
  }
  sync();
  control_solve<false>(c, kp->flags & MX_FLAG_POLICY_FIRST, ctrl);
  sync();
  if (lane < on) d.osc_tau[on * ww + lane] = dbl[L.tau + lane];
  if (lane < 3) d.osc_goal_pos[3 * ww + lane] = dbl[L.goalpos + lane];
  if (lane < 9) d.osc_goal_rot[9 * ww + lane] = dbl[L.goalrot + lane];
  if (lane < 2) d.osc_gripper[2 * ww + lane] = dbl[L.grip + lane];
  if (lane < 3) d.osc_rank[3 * ww + lane] = misc[kRank0 + lane];
  if (lane == 0) d.osc_error[ww] = misc[kCtrlErr];
  for (int a = lane; a < nu; a += kLanes) d.ctrl[ww * nu + a] = ctrl[a];
}

int osc_launch(const MxModel* m, const MxData* d, int flags, void* stream) {
  const int rc = mx_check(m, d);
  if (rc) return rc;
  const OscParams a{*m, *d, make_layout(*m), flags};
  const size_t shared = (size_t)a.L.otmp_end * sizeof(double) + 16 * sizeof(int) + (size_t)m->nu * sizeof(float);
  hipLaunchKernelGGL(osc_kernel, dim3(d->nworld), dim3(kLanes), shared, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

// ---- observation sampling outside the control step (after a reset), and its reset
struct ObsParams {
  MxData d;
  MxObsPlan obs;
  const int32_t* mask;
  int nq, nv, nsite, nbody;
  real dt;
  int force;
};

// One wavefront per world, reading the published fields in HBM.
__global__ __launch_bounds__(kLanes) void observe_kernel(ObsParams a) {
  const int w = blockIdx.x;
  if (w >= a.d.nworld || (a.mask && !a.mask[w])) return;
  const size_t ww = (size_t)w;
  const real* qp = a.d.qpos + ww * a.nq;
  const real* qv = a.d.qvel + ww * a.nv;
  const real* sx = a.d.site_xpos + ww * 3 * a.nsite;
  const real* bx = a.d.xpos + ww * 3 * a.nbody;
  const real* bq = a.d.xquat + ww * 4 * a.nbody;
  const int nq = a.nq, nv = a.nv, ns3 = 3 * a.nsite, nb3 = 3 * a.nbody, nb4 = 4 * a.nbody;
  typedef const __attribute__((address_space(4))) ObsParams KObs;
  KObs& k = *(KObs*)__builtin_amdgcn_kernarg_segment_ptr();
  obs_sample(k.obs, ww, (int)threadIdx.x, a.dt, a.force, [&](int code) {
    const int e = code & 0xffffff;
    switch (code >> 24) {
      case MX_OBS_SRC_QPOS: return e < nq ? qp[e] : 0.f;
      case MX_OBS_SRC_QVEL: return e < nv ? qv[e] : 0.f;
      case MX_OBS_SRC_SITE_XPOS: return e < ns3 ? sx[e] : 0.f;
      case MX_OBS_SRC_XPOS: return e < nb3 ? bx[e] : 0.f;
      case MX_OBS_SRC_XQUAT: return e < nb4 ? bq[e] : 0.f;
      default: return 0.f;
    }
  });
}

// elapsed, present, cache, observed and sidequat of the masked worlds to zero (sampled kept)
__global__ __launch_bounds__(kLanes) void observe_reset_kernel(MxObsPlan p, int nworld, const int32_t* mask) {
  const int w = blockIdx.x;
  if (w >= nworld || (mask && !mask[w])) return;
  const size_t ww = (size_t)w;
  for (int s = threadIdx.x; s < p.nspec; s += kLanes) {
    p.elapsed[ww * p.nspec + s] = 0.f;
    p.present[ww * p.nspec + s] = 0;
  }
  for (int j = threadIdx.x; j < p.width; j += kLanes) {
    p.cache[ww * p.width + j] = 0.f;
    p.observed[ww * p.width + j] = 0.f;
    p.sidequat[ww * p.width + j] = 0.f;
  }
}

// A plan the kernels can index: counts in range and every pointer set (the device arrays' contents
// are bounds-checked where the kernels read them).
int obs_check(const MxObsPlan* p) {
  if (!p || p->nspec < 1 || p->nspec > MX_OBS_MAX_SPECS || p->width < 1) return MX_ERR_INVALID;
  const void* need[] = {p->op, p->offset, p->size, p->index_offset, p->indices, p->dep0, p->dep1, p->dep2,
                        p->presence, p->enabled, p->period, p->cache, p->observed, p->sidequat, p->elapsed,
                        p->sampled, p->present, p->events};
  for (const void* q : need)
    if (!q) return MX_ERR_INVALID;
  return 0;
}
}  // namespace mx
#elif defined(MX_SLAB)
namespace MX_NS {
size_t slab_bytes_for(const MxModel* m) { return slab_bytes(make_layout(*m)); }
}  // namespace MX_NS
#endif

#if !defined(MX_SLAB) && !defined(MX_F64)
extern "C" {

int mx_abi_version(void) { return MX_ABI_VERSION; }
size_t mx_model_bytes(void) { return sizeof(MxModel); }
size_t mx_data_bytes(void) { return sizeof(MxData); }
int mx_arch(void) { return 950; }
const char* mx_source_id(void) { return "mx_step.hip:world-local-v8"; }

int mx_field_count(int which) { return which < 0 || which > 6 ? -1 : mx::count_names(which); }
const char* mx_field_name(int which, int index) {
  if (which < 0 || which > 6 || index < 0 || index >= mx::count_names(which)) return nullptr;
  return mx::kFieldTables[which][index];
}

int mx_check(const MxModel* m, const MxData* d) {
  if (!m || !d) return MX_ERR_INVALID;
  if (m->abi_version != MX_ABI_VERSION) return MX_ERR_INVALID;
  if (d->nworld < 1 || m->nq < 1 || m->nv < 1 || m->nbody < 2 || m->nsite < 1 || m->ntree < 1)
    return MX_ERR_INVALID;
  if (m->osc_ndof < 1 || m->osc_ndof > MX_OSC_MAXDOF || m->nu < m->osc_ndof + 2) return MX_ERR_DOMAIN;
  if (m->nlevel < 1 || m->nM < 1 || m->nMpair < m->nv) return MX_ERR_INVALID;
  if (m->osc_site < 0 || m->osc_site >= m->nsite) return MX_ERR_INVALID;
  if (m->nbody > 1023 || m->nv > 1023 || m->nM > 1023 || m->maxtree > 63 || m->maxchain < 1) return MX_ERR_DOMAIN;
  if (m->nMdamp < 0 || m->nM + m->nMdamp > 1023) return MX_ERR_DOMAIN;
  if (m->njmax < 0 || m->njmax > 16384 || m->nconmax < 0 || m->ntree > 255) return MX_ERR_DOMAIN;
  if (m->njmax > 0 && (m->nconmax < 1 || m->maxpairdof < 1 || m->opt_cone < 0 || m->opt_cone > 1)) return MX_ERR_DOMAIN;
  // force / torque sensors: three values each
  if (m->nsensor < 0 || m->nsensor > 1024 || m->nsensordata < 3 * m->nsensor) return MX_ERR_DOMAIN;
  if (m->nsensor > 0 && !d->sensordata) return MX_ERR_INVALID;
  if (m->njmax == 0 && !(m->opt_disableflags & 1)) return MX_ERR_DOMAIN;
  // every model array (an array of zero length may point anywhere valid: the kernels index it by
  // the model's counts only)
#define MX_NONNULL(name) if (!m->name) return MX_ERR_INVALID;
  MX_MODEL_REAL_ARRAYS(MX_NONNULL)
  MX_MODEL_INT_ARRAYS(MX_NONNULL)
#undef MX_NONNULL
  // the per-world state, derived fields and controller arrays every launch reads or writes
  const void* need[] = {d->time, d->qpos, d->qvel, d->ctrl, d->qacc_warmstart, d->qfrc_applied, d->qacc,
                        d->qacc_smooth, d->qfrc_bias, d->qfrc_passive, d->qfrc_actuator, d->qfrc_smooth,
                        d->qfrc_constraint, d->actuator_force, d->M, d->xpos, d->xquat, d->xmat,
                        d->geom_xpos, d->geom_xmat, d->site_xpos, d->site_xmat, d->subtree_com,
                        d->osc_mass, d->osc_jac, d->osc_q, d->osc_qvel, d->osc_bias, d->osc_ee_pos,
                        d->osc_ee_rot, d->osc_ee_vel, d->osc_action, d->osc_goal_pos, d->osc_goal_rot,
                        d->osc_gripper, d->osc_gains, d->osc_q0, d->osc_tau, d->overflow, d->osc_error,
                        d->osc_rank, d->nstep, d->xfrc_applied, d->cacc, d->cfrc_int, d->cfrc_ext};
  for (const void* p : need)
    if (!p) return MX_ERR_INVALID;
  if (m->osc_action_scaled < 0 || m->osc_action_scaled > 1) return MX_ERR_INVALID;
  if (m->osc_action_scaled && !d->osc_action_scale) return MX_ERR_INVALID;
  // contacts, rows and their counts, published whenever the model has constraint rows
  if (m->njmax > 0) {
    const void* rows[] = {d->ncon, d->nefc, d->solver_niter, d->stat_sums, d->contact_pos, d->contact_frame, d->contact_dist,
                          d->contact_friction, d->contact_includemargin, d->contact_geom, d->contact_dim,
                          d->efc_force, d->efc_pos, d->efc_D, d->efc_aref, d->efc_type, d->efc_state, d->efc_id};
    for (const void* p : rows)
      if (!p) return MX_ERR_INVALID;
    if (m->has_body_active && !d->body_active) return MX_ERR_INVALID;
  }
  // a working set beyond the LDS of a workgroup needs the workspace slabs
  if (mx::make_layout(*m).bytes > MX_LDS_BUDGET && !mx::workspace_ok(m, d)) return MX_ERR_LDS;
  return 0;
}

int mx_lds_bytes(const MxModel* m) { return m ? mx::make_layout(*m).bytes : MX_ERR_INVALID; }

int mx_lds_bytes_fp64(const MxModel* m) { return m ? mx_f64::lds_bytes_for(m) : MX_ERR_INVALID; }

size_t mx_workspace_bytes(const MxModel* m) { return m ? mx_slab::slab_bytes_for(m) : 0; }

int mx_control_step(const MxModel* m, const MxData* d, int substeps, int flags, void* stream) {
  return mx::launch(m, d, nullptr, substeps, flags & ~MX_FLAG_NO_INTEGRATE, stream);
}

int mx_forward(const MxModel* m, const MxData* d, const int32_t* mask, int flags, void* stream) {
  return mx::launch(m, d, mask, 1, (flags | MX_FLAG_NO_INTEGRATE) & ~MX_FLAG_POLICY_FIRST, stream);
}

int mx_control_step_noalloc(const MxModel* m, const MxData* d, int substeps, int flags, void* stream) {
  return mx::control_step_noalloc(m, d, substeps, flags, stream);
}

size_t mx_obs_plan_bytes(void) { return sizeof(MxObsPlan); }

int mx_osc(const MxModel* m, const MxData* d, int flags, void* stream) { return mx::osc_launch(m, d, flags, stream); }

int mx_control_step_observed(const MxModel* m, const MxData* d, const MxObsPlan* plan, int substeps, int flags,
                             void* stream) {
  const int rc = mx::obs_check(plan);
  if (rc) return rc;
  return mx::launch(m, d, nullptr, substeps, flags & ~MX_FLAG_NO_INTEGRATE, stream, plan);
}

int mx_observe(const MxModel* m, const MxData* d, const MxObsPlan* plan, const int32_t* mask, float dt, int force,
               void* stream) {
  int rc = mx_check(m, d);
  if (rc) return rc;
  if ((rc = mx::obs_check(plan))) return rc;
  if (!(dt > 0.f) || !std::isfinite(dt)) return MX_ERR_INVALID;
  const mx::ObsParams a{*d, *plan, mask, m->nq, m->nv, m->nsite, m->nbody, dt, force};
  hipLaunchKernelGGL(mx::observe_kernel, dim3(d->nworld), dim3(mx::kLanes), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int mx_observe_reset(const MxData* d, const MxObsPlan* plan, const int32_t* mask, void* stream) {
  if (!d || d->nworld < 1) return MX_ERR_INVALID;
  const int rc = mx::obs_check(plan);
  if (rc) return rc;
  hipLaunchKernelGGL(mx::observe_reset_kernel, dim3(d->nworld), dim3(mx::kLanes), 0, (hipStream_t)stream, *plan,
                     d->nworld, mask);
  return (int)hipGetLastError();
}

const char* mx_error_string(int code) {
  switch (code) {
    case 0: return "success";
    case MX_ERR_INVALID: return "invalid argument";
    case MX_ERR_DOMAIN: return "model outside the admitted domain";
    case MX_ERR_LDS: return "per-world working set exceeds the LDS budget and no (or too small a) workspace is given";
    case MX_ERR_SCRATCH: return "the batch's workspace slabs exceed the library's fixed device scratch (MX_SCRATCH_BYTES per device)";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}
}
#endif  // MX_SLAB
