// Narrowphase routines for the world-local kernel (FP32, one lane per candidate pair).
//
// Same geometric algorithms as the CPU oracle (oracle/oracle_collision.cpp), written for a single
// lane with register-resident state.  Reference leaves restated: plane-sphere / capsule / box
// gpu/cuda/collision/mjwarp_plane.cu:18-39, sphere-box mjwarp_box.cu:14-32, capsule-box
// mjwarp_box.cu:33-102, box-box SAT + edge contact or clipped face mjwarp_box.cu:103-176.
// Capsule-capsule and sphere-capsule have no port in the reference (MuJoCo semantics here).
// Convention: the normal points from geom1 to geom2, pos is the midpoint between the surfaces,
// dist < 0 is penetration.  `thr` arguments are the detection threshold margin + gap.
// Provenance: the routines restated here follow reference files headed "Copyright 2025 The Newton
// Developers, SPDX-License-Identifier: Apache-2.0" (MJWarp-derived CUDA in gpu/cuda/collision/);
// their feature selection, tolerances and step order are kept so that the contact sets match.
#pragma once
#include <hip/hip_runtime.h>
#include "mx_math.h"

namespace MX_NS {

enum GeomType : int { GT_PLANE = 0, GT_SPHERE = 2, GT_CAPSULE = 3, GT_BOX = 6, GT_MESH = 7 };

constexpr int kMaxPairContacts = 8;   // clipped box face: up to 8 points; plane-box: 8 corners

struct GeomX {
  int type;
  real pos[3], mat[9], size[3];
  const sfloat* vert;  // mesh vertices (LDS: the image, or the window copy), local frame
  int nvert, mesh;     // mesh id (-1: not a mesh)
};

struct RawOut {        // contacts of one pair
  int n;
  unsigned tangent_mask;   // bit k: contact k fixes its second frame axis (plane-capsule)
  real pos[kMaxPairContacts][3], normal[kMaxPairContacts][3], dist[kMaxPairContacts];
  real tangent[3];
};

__device__ __forceinline__ real dot3f(const real* a, const real* b) { return a[0] * b[0] + a[1] * b[1] + a[2] * b[2]; }
__device__ __forceinline__ real norm3f(const real* a) { return r_sqrt(dot3f(a, a)); }
__device__ __forceinline__ void axisf(const real* mat, int k, real* o) { o[0] = mat[k]; o[1] = mat[3 + k]; o[2] = mat[6 + k]; }
__device__ __forceinline__ void mulmtv3(const real* m, const real* v, real* r) {
  real a = m[0] * v[0] + m[3] * v[1] + m[6] * v[2];
  real b = m[1] * v[0] + m[4] * v[1] + m[7] * v[2];
  real c = m[2] * v[0] + m[5] * v[1] + m[8] * v[2];
  r[0] = a; r[1] = b; r[2] = c;
}

__device__ __forceinline__ void raw_push(RawOut& __restrict__ o, const real* pos, const real* n, real dist) {
  if (o.n >= kMaxPairContacts) return;
  for (int k = 0; k < 3; ++k) { o.pos[o.n][k] = pos[k]; o.normal[o.n][k] = n[k]; }
  o.dist[o.n] = dist;
  ++o.n;
}

// MJWarp make_frame: tangent from y (or z when the normal is close to y), then the cross product.
__device__ inline void make_frame(const real* n, real* frame) {
  real a[3] = {n[0], n[1], n[2]};
  real l = norm3f(a);
  if (l > 1e-15f) { a[0] /= l; a[1] /= l; a[2] /= l; }
  real b[3];
  if (-0.5f < a[1] && a[1] < 0.5f) { b[0] = 0.f; b[1] = 1.f; b[2] = 0.f; }
  else { b[0] = 0.f; b[1] = 0.f; b[2] = 1.f; }
  real d = dot3f(a, b);
  for (int k = 0; k < 3; ++k) b[k] -= a[k] * d;
  l = norm3f(b);
  if (l > 1e-15f) { b[0] /= l; b[1] /= l; b[2] /= l; }
  real c[3];
  cross3(a, b, c);
  for (int k = 0; k < 3; ++k) { frame[k] = a[k]; frame[3 + k] = b[k]; frame[6 + k] = c[k]; }
}

// ---------------------------------------------------------------- plane
__device__ inline void plane_point(const GeomX& __restrict__ p, const real* c, real r, real thr, RawOut& __restrict__ o) {
  real n[3];
  axisf(p.mat, 2, n);
  real d[3] = {c[0] - p.pos[0], c[1] - p.pos[1], c[2] - p.pos[2]};
  real dist = dot3f(n, d) - r;
  if (!(dist < thr)) return;
  real pos[3];
  for (int k = 0; k < 3; ++k) pos[k] = c[k] - n[k] * (r + 0.5f * dist);
  raw_push(o, pos, n, dist);
}

// both end spheres, +axis end first; frame axis 2 = capsule axis projected on the plane
__device__ inline void plane_capsule(const GeomX& __restrict__ p, const GeomX& __restrict__ cap, real thr, RawOut& __restrict__ o) {
  real n[3], ax[3];
  axisf(p.mat, 2, n);
  axisf(cap.mat, 2, ax);
  real proj = dot3f(n, ax);
  real b[3] = {ax[0] - n[0] * proj, ax[1] - n[1] * proj, ax[2] - n[2] * proj};
  real len = norm3f(b);
  if (len != 0.f) { b[0] /= len; b[1] /= len; b[2] /= len; }
  if (len < 0.5f) {
    bool y = -0.5f < n[1] && n[1] < 0.5f;
    b[0] = 0.f; b[1] = y ? 1.f : 0.f; b[2] = y ? 0.f : 1.f;
  }
  for (int k = 0; k < 3; ++k) o.tangent[k] = b[k];
  for (int e = 1; e >= -1; e -= 2) {
    real c[3];
    for (int k = 0; k < 3; ++k) c[k] = cap.pos[k] + real(e) * ax[k] * cap.size[1];
    int before = o.n;
    plane_point(p, c, cap.size[0], thr, o);
    if (o.n > before) o.tangent_mask |= 1u << before;
  }
}

// every box corner under the threshold, in corner order
__device__ inline void plane_box(const GeomX& __restrict__ p, const GeomX& __restrict__ box, real thr, RawOut& __restrict__ o) {
  real n[3];
  axisf(p.mat, 2, n);
  real dc[3] = {box.pos[0] - p.pos[0], box.pos[1] - p.pos[1], box.pos[2] - p.pos[2]};
  real center_dist = dot3f(dc, n);
  for (int i = 0; i < 8; ++i) {
    real l[3] = {(i & 1) ? box.size[0] : -box.size[0], (i & 2) ? box.size[1] : -box.size[1],
                  (i & 4) ? box.size[2] : -box.size[2]};
    real corner[3];
    mulmv3(box.mat, l, corner);
    real dist = center_dist + dot3f(n, corner);
    if (!(dist < thr)) continue;
    real pos[3];
    for (int k = 0; k < 3; ++k) pos[k] = corner[k] + box.pos[k] - 0.5f * n[k] * dist;
    raw_push(o, pos, n, dist);
  }
}

// Convex mesh against a plane (plane_mesh, gpu/cuda/collision/mjwarp_plane.cu:80-121): the support
// vertex along the plane's inward normal; when it lies within the threshold, up to three more
// corners of the incident hull polygon whose normal is most opposed to the plane normal (chosen by
// hull4, mjwarp_plane.cu:58-79: the largest quadrilateral grown from that vertex), those not above
// the geom centre.  Polygons come from the model arrays in device memory (this path is rare).
__device__ inline real poly_quad_area(const GeomX& __restrict__ g, const int* pv, int i, int j, int k, int l) {
  v4f a = *(const sfloat4*)(g.vert + 4 * pv[i]), b = *(const sfloat4*)(g.vert + 4 * pv[j]);
  v4f c = *(const sfloat4*)(g.vert + 4 * pv[k]), d = *(const sfloat4*)(g.vert + 4 * pv[l]);
  real u[3] = {a.x - c.x, a.y - c.y, a.z - c.z}, v[3] = {b.x - d.x, b.y - d.y, b.z - d.z}, x[3];
  cross3(u, v, x);
  return 0.5f * r_sqrt(dot3f(x, x));
}

__device__ inline void plane_mesh(KModel& m, const GeomX& __restrict__ p, const GeomX& __restrict__ g, real thr, RawOut& __restrict__ o) {
  real n[3], ln[3];
  axisf(p.mat, 2, n);
  for (int k = 0; k < 3; ++k) ln[k] = g.mat[k] * n[0] + g.mat[3 + k] * n[1] + g.mat[6 + k] * n[2];
  int index = -1;
  real best = -1e10f;
  for (int i = 0; i < g.nvert; ++i) {
    v4f q = *(const sfloat4*)(g.vert + 4 * i);
    real s = -(ln[0] * q.x + ln[1] * q.y + ln[2] * q.z);
    if (s > best) { best = s; index = i; }
  }
  if (index < 0) return;
  auto world = [&](int i, real* w) {
    v4f q = *(const sfloat4*)(g.vert + 4 * i);
    real l[3] = {q.x, q.y, q.z};
    mulmv3(g.mat, l, w);
    for (int k = 0; k < 3; ++k) w[k] += g.pos[k];
  };
  auto emit = [&](const real* v) {
    real d[3] = {v[0] - p.pos[0], v[1] - p.pos[1], v[2] - p.pos[2]}, dist = dot3f(n, d), pos[3];
    for (int k = 0; k < 3; ++k) pos[k] = v[k] - 0.5f * dist * n[k];
    if (dist < thr) raw_push(o, pos, n, dist);
    return dist;
  };
  real v0[3];
  world(index, v0);
  real dist = emit(v0);
  const int mesh = g.mesh, padr = m.mesh_polyadr[mesh], vadr = m.mesh_vertadr[mesh];
  if (m.mesh_polynum[mesh] <= 0 || dist > thr) return;
  int best_poly = -1;
  real best_dot = 1.f;
  const int madr = m.mesh_polymapadr[vadr + index], mnum = m.mesh_polymapnum[vadr + index];
  for (int i = 0; i < mnum; ++i) {
    int id = m.mesh_polymap[madr + i];
    const float* pn = m.mesh_polynormal + 3 * (padr + id);
    real dt = pn[0] * ln[0] + pn[1] * ln[1] + pn[2] * ln[2];
    if (dt < best_dot) { best_dot = dt; best_poly = id; }
  }
  if (best_poly < 0) return;
  const int* pv = m.mesh_polyvert + m.mesh_polyvertadr[padr + best_poly];
  const int count = m.mesh_polyvertnum[padr + best_poly];
  int anchor = 0;
  for (int i = 0; i < count; ++i)
    if (pv[i] == index) { anchor = i; break; }
  int b = (anchor + 1) % count, c = (anchor + 2) % count, d = (anchor + 3) % count;
  int idx[4] = {anchor, b, c, d}, hull = count;
  if (count > 4) {
    hull = 4;
    real area = poly_quad_area(g, pv, anchor, b, c, d);
    while (true) {
      int next = (d + 1) % count;
      real cand = poly_quad_area(g, pv, anchor, b, c, next);
      if (cand <= area) break;
      d = next; area = cand; idx[1] = b; idx[2] = c; idx[3] = d;
      while (true) {
        next = (c + 1) % count;
        cand = poly_quad_area(g, pv, anchor, b, next, d);
        if (cand <= area) break;
        c = next; area = cand; idx[1] = b; idx[2] = c; idx[3] = d;
      }
      while (true) {
        next = (b + 1) % count;
        cand = poly_quad_area(g, pv, anchor, next, c, d);
        if (cand <= area) break;
        b = next; area = cand; idx[1] = b; idx[2] = c; idx[3] = d;
      }
    }
  }
  for (int i = 1; i < hull; ++i) {
    real v[3];
    world(pv[idx[i]], v);
    real up[3] = {v[0] - g.pos[0], v[1] - g.pos[1], v[2] - g.pos[2]};
    if (dot3f(n, up) > 0.f) continue;
    emit(v);
  }
}

__device__ __forceinline__ void segment_ends(const GeomX& __restrict__ g, real* a, real* b) {
  real ax[3];
  axisf(g.mat, 2, ax);
  for (int k = 0; k < 3; ++k) { a[k] = g.pos[k] - g.size[1] * ax[k]; b[k] = g.pos[k] + g.size[1] * ax[k]; }
}

// ---------------------------------------------------------------- spheres and segments
__device__ inline void sphere_sphere(const real* c1, real r1, const real* c2, real r2, real margin,
                                     RawOut& __restrict__ o, const real* fallback) {
  real d[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
  real len = norm3f(d);
  real dist = len - r1 - r2;
  if (dist >= margin) return;
  real n[3];
  if (len > 1e-15f) { for (int k = 0; k < 3; ++k) n[k] = d[k] / len; }
  else { for (int k = 0; k < 3; ++k) n[k] = fallback[k]; }
  real pos[3];
  for (int k = 0; k < 3; ++k) pos[k] = c1[k] + n[k] * (r1 + 0.5f * dist);
  raw_push(o, pos, n, dist);
}

__device__ inline void closest_segments(const real* p1, const real* q1, const real* p2, const real* q2,
                                        real& s, real& t) {
  real d1[3], d2[3], r[3];
  for (int k = 0; k < 3; ++k) { d1[k] = q1[k] - p1[k]; d2[k] = q2[k] - p2[k]; r[k] = p1[k] - p2[k]; }
  real a = dot3f(d1, d1), e = dot3f(d2, d2), f = dot3f(d2, r);
  const real tiny = 1e-15f;
  if (a <= tiny && e <= tiny) { s = t = 0.f; return; }
  if (a <= tiny) { s = 0.f; t = r_min(r_max(f / e, 0.f), 1.f); return; }
  real c = dot3f(d1, r);
  if (e <= tiny) { t = 0.f; s = r_min(r_max(-c / a, 0.f), 1.f); return; }
  real b = dot3f(d1, d2), denom = a * e - b * b;
  s = denom > tiny * a * e ? r_min(r_max((b * f - c * e) / denom, 0.f), 1.f) : 0.f;
  t = (b * s + f) / e;
  if (t < 0.f) { t = 0.f; s = r_min(r_max(-c / a, 0.f), 1.f); }
  else if (t > 1.f) { t = 1.f; s = r_min(r_max((b - c) / a, 0.f), 1.f); }
}

__device__ inline void capsule_capsule(const GeomX& __restrict__ g1, const GeomX& __restrict__ g2, real margin, RawOut& __restrict__ o) {
  real a1[3], b1[3], a2[3], b2[3];
  segment_ends(g1, a1, b1);
  segment_ends(g2, a2, b2);
  real r1 = g1.size[0], r2 = g2.size[0];
  real d1[3], d2[3], cr[3];
  for (int k = 0; k < 3; ++k) { d1[k] = b1[k] - a1[k]; d2[k] = b2[k] - a2[k]; }
  cross3(d1, d2, cr);
  real l1 = norm3f(d1), l2 = norm3f(d2);
  real fb[3] = {cr[0], cr[1], cr[2]};
  real lf = norm3f(fb);
  if (lf < 1e-15f) { fb[0] = 0.f; fb[1] = 0.f; fb[2] = 1.f; }
  else { fb[0] /= lf; fb[1] /= lf; fb[2] /= lf; }
  if (l1 > 1e-15f && l2 > 1e-15f && norm3f(cr) < 1e-3f * l1 * l2) {
    real u[3] = {d1[0] / l1, d1[1] / l1, d1[2] / l1};
    real ta[3] = {a2[0] - a1[0], a2[1] - a1[1], a2[2] - a1[2]}, tb[3] = {b2[0] - a1[0], b2[1] - a1[1], b2[2] - a1[2]};
    real s0 = dot3f(ta, u), s1 = dot3f(tb, u);
    real lo = r_max(r_min(s0, s1), 0.f), hi = r_min(r_max(s0, s1), l1);
    if (hi - lo > 1e-6f * l1) {
      for (int e = 0; e < 2; ++e) {
        real sp = e == 0 ? lo : hi;
        real p1[3], p2[3];
        for (int k = 0; k < 3; ++k) p1[k] = a1[k] + u[k] * sp;
        real t = r_min(r_max((sp - s0) / (s1 - s0), 0.f), 1.f);
        for (int k = 0; k < 3; ++k) p2[k] = a2[k] + d2[k] * t;
        sphere_sphere(p1, r1, p2, r2, margin, o, fb);
      }
      return;
    }
  }
  real s, t;
  closest_segments(a1, b1, a2, b2, s, t);
  real p1[3], p2[3];
  for (int k = 0; k < 3; ++k) { p1[k] = a1[k] + d1[k] * s; p2[k] = a2[k] + d2[k] * t; }
  sphere_sphere(p1, r1, p2, r2, margin, o, fb);
}

// ---------------------------------------------------------------- sphere / capsule / box
constexpr real kBoxMin = 1e-15f, kBoxMax = 1e10f;
__device__ __forceinline__ real clampf(real v, real lo, real hi) { return r_max(lo, r_min(hi, v)); }
__device__ __forceinline__ real safe_divf(real x, real y) { return x / (y != 0.f ? y : kBoxMin); }

// sphere (centre c, radius r) as geom 1 against box geom 2
__device__ inline void sphere_box(const real* c, real r, const GeomX& __restrict__ box, real thr, RawOut& __restrict__ o) {
  real d[3] = {c[0] - box.pos[0], c[1] - box.pos[1], c[2] - box.pos[2]}, local[3], clamped[3];
  mulmtv3(box.mat, d, local);
  for (int k = 0; k < 3; ++k) clamped[k] = clampf(local[k], -box.size[k], box.size[k]);
  real dir[3] = {clamped[0] - local[0], clamped[1] - local[1], clamped[2] - local[2]};
  real len = r_sqrt(dot3f(dir, dir));
  if (len != 0.f) { real inv = 1.f / len; dir[0] *= inv; dir[1] *= inv; dir[2] *= inv; }
  real lpos[3], ln[3], dist;
  if (len <= kBoxMin) {
    real closest = 2.f * (box.size[0] + box.size[1] + box.size[2]);
    int face = 0;
    for (int i = 0; i < 6; ++i) {
      real f = r_abs(((i % 2) ? 1.f : -1.f) * box.size[i / 2] - local[i / 2]);
      if (closest > f) { closest = f; face = i; }
    }
    for (int k = 0; k < 3; ++k) ln[k] = 0.f;
    ln[face / 2] = (face % 2) ? -1.f : 1.f;
    for (int k = 0; k < 3; ++k) lpos[k] = local[k] + ln[k] * (r - closest) * 0.5f;
    dist = -closest - r;
  } else {
    for (int k = 0; k < 3; ++k) { lpos[k] = 0.5f * (clamped[k] + local[k] + dir[k] * r); ln[k] = dir[k]; }
    dist = len - r;
  }
  if (!(dist < thr)) return;
  real wpos[3], n[3];
  mulmv3(box.mat, lpos, wpos);
  mulmv3(box.mat, ln, n);
  for (int k = 0; k < 3; ++k) wpos[k] += box.pos[k];
  raw_push(o, wpos, n, dist);
}

// capsule geom 1 against box geom 2: closest feature pair (end caps, then the 12 box edges in
// corner-major order), a sphere contact there and possibly a second one along the segment
__device__ __forceinline__ void capsule_box(const GeomX& __restrict__ cap, const GeomX& __restrict__ box, real thr, RawOut& __restrict__ o) {
  real radius = cap.size[0], half = cap.size[1];
  real d[3] = {cap.pos[0] - box.pos[0], cap.pos[1] - box.pos[1], cap.pos[2] - box.pos[2]}, pos[3], wax[3], ax[3];
  mulmtv3(box.mat, d, pos);
  axisf(cap.mat, 2, wax);
  mulmtv3(box.mat, wax, ax);
  const real* size = box.size;
  real ha[3] = {ax[0] * half, ax[1] * half, ax[2] * half};
  int axisdir = int(ha[0] > 0.f) + 2 * int(ha[1] > 0.f) + 4 * int(ha[2] > 0.f);
  real bestdist = 1e32f, bestsegment = -12.f, bestbox = 0.f;
  int type = -4, face = -12, corner = -123, edge = -123;
  for (int i = -1; i <= 1; i += 2) {
    real tip[3], pt[3];
    int outside = 0, a = -1;
    for (int k = 0; k < 3; ++k) { tip[k] = pos[k] + real(i) * ha[k]; pt[k] = tip[k]; }
    for (int j = 0; j < 3; ++j) {
      if (pt[j] < -size[j]) { ++outside; a = j; pt[j] = -size[j]; }
      else if (pt[j] > size[j]) { ++outside; a = j; pt[j] = size[j]; }
    }
    if (outside > 1) continue;
    real dif[3] = {pt[0] - tip[0], pt[1] - tip[1], pt[2] - tip[2]};
    real dd = dot3f(dif, dif);
    if (dd < bestdist) { bestdist = dd; bestsegment = real(i); type = -2 + i; face = a; }
  }
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 3; ++j) {
      if (i & (1 << j)) continue;
      real pt[3] = {(i & 1) ? size[0] : -size[0], (i & 2) ? size[1] : -size[1], (i & 4) ? size[2] : -size[2]};
      pt[j] = 0.f;
      real dif[3] = {pt[0] - pos[0], pt[1] - pos[1], pt[2] - pos[2]};
      real u = -size[j] * dif[j], v = dot3f(ha, dif), ma = size[j] * size[j], mb = -size[j] * ha[j], mc = half * half;
      real det = ma * mc - mb * mb;
      if (r_abs(det) < kBoxMin) continue;
      real inv = 1.f / det, x1 = (mc * u - mb * v) * inv, x2 = (ma * v - mb * u) * inv;
      int s1 = 1, s2 = 1;
      if (x1 > 1.f) { x1 = 1.f; s1 = 2; x2 = safe_divf(v - mb, mc); }
      else if (x1 < -1.f) { x1 = -1.f; s1 = 0; x2 = safe_divf(v + mb, mc); }
      bool over = x2 > 1.f;
      if (over || x2 < -1.f) {
        if (over) { x2 = 1.f; s2 = 2; x1 = safe_divf(u - mb, ma); }
        else { x2 = -1.f; s2 = 0; x1 = safe_divf(u + mb, ma); }
        if (x1 > 1.f) { x1 = 1.f; s1 = 2; }
        else if (x1 < -1.f) { x1 = -1.f; s1 = 0; }
      }
      for (int k = 0; k < 3; ++k) dif[k] -= ha[k] * x2;
      dif[j] += size[j] * x1;
      real dd = dot3f(dif, dif);
      int config = s1 * 3 + s2;
      if (dd < bestdist - kBoxMin) {
        bestdist = dd; bestsegment = x2; bestbox = x1;
        corner = i + (1 << j) * (config / 6); edge = j; type = config;
      }
    }
  if (type == -4) return;
  real second = -4.f;
  if (type >= 0 && type / 3 != 1) {
    int config = axisdir ^ corner;
    if (config != 0 && config != 7) {
      real mul;
      if (config == 1 || config == 2 || config == 4) mul = 1.f;
      else { mul = -1.f; config = 7 - config; }
      int a = config == 1 ? 0 : config == 2 ? 1 : 2, a1 = (a + 1) % 3, a2 = (a + 2) % 3;
      if (ax[a] * ax[a] > 0.5f) {
        real mm = 2.f * safe_divf(size[a], r_abs(ha[a]));
        second = r_min(1.f - mul * bestsegment, mm);
      } else {
        real mm = 2.f * r_min(safe_divf(size[a1], r_abs(ha[a1])), safe_divf(size[a2], r_abs(ha[a2])));
        second = -r_min(1.f + mul * bestsegment, mm);
      }
      second *= mul;
    }
  } else if (type >= 0 && type / 3 == 1) {
    int config = (axisdir ^ corner) & (7 - (1 << edge));
    if (config == 1 || config == 2 || config == 4) {
      int a = edge, a1 = (edge + 1) % 3, a2 = (edge + 2) % 3;
      if (r_abs(ax[a1]) > r_abs(ax[a2])) a1 = a2;
      a2 = 3 - a - a1;
      real mul;
      if (config & (1 << a2)) { mul = 1.f; second = 1.f - bestsegment; }
      else { mul = -1.f; second = 1.f + bestsegment; }
      real e1 = 2.f * safe_divf(size[a2], r_abs(ha[a2]));
      second = r_min(e1, second);
      real e2 = (bool(axisdir & (1 << a)) == bool(config & (1 << a2))) ? 1.f - bestbox : 1.f + bestbox;
      e1 = size[a] * safe_divf(e2, r_abs(ha[a]));
      second = r_min(e1, second);
      second *= mul;
    }
  } else if (type < 0 && face != -1) {
    real mul = type == -3 ? 1.f : -1.f;
    second = 2.f;
    real tmp[3] = {pos[0] - ha[0] * mul, pos[1] - ha[1] * mul, pos[2] - ha[2] * mul};
    for (int i = 0; i < 3; ++i) {
      if (i == face) continue;
      real inv = safe_divf(mul, ha[i]);
      real e1 = (size[i] - tmp[i]) * inv;
      if (0.f < e1 && e1 < second) second = e1;
      e1 = (-size[i] - tmp[i]) * inv;
      if (0.f < e1 && e1 < second) second = e1;
    }
    second *= mul;
  }
  for (int q = 0; q < (second > -3.f ? 2 : 1); ++q) {
    real t = q == 0 ? bestsegment : second + bestsegment;
    real l[3] = {pos[0] + ha[0] * t, pos[1] + ha[1] * t, pos[2] + ha[2] * t}, w[3];
    mulmv3(box.mat, l, w);
    for (int k = 0; k < 3; ++k) w[k] += box.pos[k];
    sphere_box(w, radius, box, thr, o);
  }
}

// ---------------------------------------------------------------- box-box
// clip the face-plane polygon against sign * p[coord] <= limit
__device__ inline int clip_face(int count, real (*poly)[3], int coord, real sign, real limit) {
  real d[8];
  bool inside = true;
  for (int i = 0; i < count; ++i) { d[i] = sign * poly[i][coord] - limit; if (!(d[i] <= 0.f)) inside = false; }
  if (inside) return count;
  real clipped[8][3];
  int n = 0;
  for (int i = 0; i < count; ++i) {
    int next = i + 1 == count ? 0 : i + 1;
    real dp = d[i], dq = d[next];
    if (dp <= 0.f && n < 8) { for (int k = 0; k < 3; ++k) clipped[n][k] = poly[i][k]; ++n; }
    if (((dp < 0.f && dq > 0.f) || (dp > 0.f && dq < 0.f)) && n < 8) {
      real t = dp / (dp - dq);
      for (int k = 0; k < 3; ++k) clipped[n][k] = poly[i][k] + t * (poly[next][k] - poly[i][k]);
      ++n;
    }
  }
  for (int i = 0; i < n; ++i) for (int k = 0; k < 3; ++k) poly[i][k] = clipped[i][k];
  return n;
}

// separating axes (3 + 3 faces, 9 edges), then one edge-edge contact or the incident face
// clipped against the reference face
__device__ __forceinline__ void box_box(const GeomX& __restrict__ g1, const GeomX& __restrict__ g2, real thr, RawOut& __restrict__ o) {
  const real *s1 = g1.size, *s2 = g2.size;
  real d21[3] = {g2.pos[0] - g1.pos[0], g2.pos[1] - g1.pos[1], g2.pos[2] - g1.pos[2]};
  real d12[3] = {-d21[0], -d21[1], -d21[2]}, pos21[3], pos12[3];
  mulmtv3(g1.mat, d21, pos21);
  mulmtv3(g2.mat, d12, pos12);
  real rot[9], ab[9];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      rot[3 * i + j] = g1.mat[i] * g2.mat[j] + g1.mat[3 + i] * g2.mat[3 + j] + g1.mat[6 + i] * g2.mat[6 + j];
      ab[3 * i + j] = r_abs(rot[3 * i + j]);
    }
  real septol = thr + 1e-6f * (s1[0] + s1[1] + s1[2] + s2[0] + s2[1] + s2[2]), best = -kBoxMax;
  int code = -1;
  for (int i = 0; i < 3; ++i) {
    real radius = ab[3 * i] * s2[0] + ab[3 * i + 1] * s2[1] + ab[3 * i + 2] * s2[2];
    real sep = r_abs(pos21[i]) - s1[i] - radius;
    if (sep > septol) return;
    if (sep > best) { best = sep; code = i; }
  }
  for (int j = 0; j < 3; ++j) {
    real radius = ab[j] * s1[0] + ab[3 + j] * s1[1] + ab[6 + j] * s1[2];
    real sep = r_abs(pos12[j]) - s2[j] - radius;
    if (sep > septol) return;
    if (sep > best) { best = sep; code = 3 + j; }
  }
  real face_best = best;
  int face_code = code;
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      int i1 = (i + 1) % 3, i2 = (i + 2) % 3;
      real x = -rot[3 * i2 + j], y = rot[3 * i1 + j], n2 = x * x + y * y;
      if (n2 < 1e-7f) continue;
      real inv = 1.f / r_sqrt(n2);
      x *= inv; y *= inv;
      real r1 = s1[i1] * r_abs(x) + s1[i2] * r_abs(y);
      int j1 = (j + 1) % 3, j2 = (j + 2) % 3;
      real a1 = x * rot[3 * i1 + j1] + y * rot[3 * i2 + j1], a2 = x * rot[3 * i1 + j2] + y * rot[3 * i2 + j2];
      real r2 = s2[j1] * r_abs(a1) + s2[j2] * r_abs(a2);
      real sep = r_abs(x * pos21[i1] + y * pos21[i2]) - r1 - r2;
      if (sep > septol) return;
      if (sep - 1e-6f * r_abs(sep) > best && sep > face_best) { best = sep; code = 6 + 3 * i + j; }
    }
  if (code < 0) return;
  int ei = 0, ej = 0, i1 = 0, i2 = 0;
  real ax[3] = {0.f, 0.f, 0.f};
  if (code >= 6) {
    ei = (code - 6) / 3; ej = (code - 6) % 3; i1 = (ei + 1) % 3; i2 = (ei + 2) % 3;
    ax[i1] = -rot[3 * i2 + ej];
    ax[i2] = rot[3 * i1 + ej];
    real l = r_sqrt(dot3f(ax, ax));
    if (l > 1e-15f) { ax[0] /= l; ax[1] /= l; ax[2] /= l; }
    real align = face_code < 3 ? r_abs(ax[face_code])
                                : r_abs(ax[0] * rot[face_code - 3] + ax[1] * rot[face_code] + ax[2] * rot[face_code + 3]);
    if (align > 0.99f && best < face_best + 0.05f * r_abs(face_best) + kBoxMin) { code = face_code; best = face_best; }
  }
  if (code >= 6) {
    int j1 = (ej + 1) % 3, j2 = (ej + 2) % 3;
    if (dot3f(ax, pos21) < 0.f) { ax[0] = -ax[0]; ax[1] = -ax[1]; ax[2] = -ax[2]; }
    real a2[3];
    mulmtv3(rot, ax, a2);
    int amb1 = -1, amb2 = -1;
    if (r_abs(ax[i1]) < 1e-5f) amb1 = i1;
    else if (r_abs(ax[i2]) < 1e-5f) amb1 = i2;
    if (r_abs(a2[j1]) < 1e-5f) amb2 = j1;
    else if (r_abs(a2[j2]) < 1e-5f) amb2 = j2;
    real dv2[3] = {rot[ej], rot[3 + ej], rot[6 + ej]};
    real b = dv2[ei], denom = 1.f - b * b, best_dist = kBoxMax;
    real w1[3] = {0.f, 0.f, 0.f}, w2[3] = {0.f, 0.f, 0.f};
    for (int v1 = 0; v1 < (amb1 >= 0 ? 2 : 1); ++v1)
      for (int v2 = 0; v2 < (amb2 >= 0 ? 2 : 1); ++v2) {
        real c1[3] = {0.f, 0.f, 0.f}, corner[3] = {0.f, 0.f, 0.f}, c2[3];
        c1[i1] = ax[i1] >= 0.f ? s1[i1] : -s1[i1];
        c1[i2] = ax[i2] >= 0.f ? s1[i2] : -s1[i2];
        if (amb1 >= 0 && v1) c1[amb1] = -c1[amb1];
        corner[j1] = a2[j1] >= 0.f ? -s2[j1] : s2[j1];
        corner[j2] = a2[j2] >= 0.f ? -s2[j2] : s2[j2];
        if (amb2 >= 0 && v2) corner[amb2] = -corner[amb2];
        mulmv3(rot, corner, c2);
        for (int k = 0; k < 3; ++k) c2[k] += pos21[k];
        real e[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
        real d1e = e[ei], d2e = dot3f(dv2, e);
        real s = denom >= kBoxMin ? (d1e - b * d2e) / denom : 0.f;
        s = clampf(s, -s1[ei], s1[ei]);
        real t = clampf(b * s - d2e, -s2[ej], s2[ej]);
        s = clampf(d1e + b * t, -s1[ei], s1[ei]);
        real q1[3] = {c1[0], c1[1], c1[2]}, q2[3];
        q1[ei] = s;
        for (int k = 0; k < 3; ++k) q2[k] = c2[k] + dv2[k] * t;
        real g[3] = {q2[0] - q1[0], q2[1] - q1[1], q2[2] - q1[2]};
        real dd = dot3f(g, g);
        if (dd < best_dist) { best_dist = dd; for (int k = 0; k < 3; ++k) { w1[k] = q1[k]; w2[k] = q2[k]; } }
      }
    real gap[3] = {w2[0] - w1[0], w2[1] - w1[1], w2[2] - w1[2]};
    real dist = dot3f(gap, ax);
    if (dist > septol || !(dist < thr)) return;
    real mid[3] = {0.5f * (w1[0] + w2[0]), 0.5f * (w1[1] + w2[1]), 0.5f * (w1[2] + w2[2])}, wpos[3], n[3];
    mulmv3(g1.mat, mid, wpos);
    for (int k = 0; k < 3; ++k) wpos[k] += g1.pos[k];
    mulmv3(g1.mat, ax, n);
    raw_push(o, wpos, n, dist);
    return;
  }
  bool ref1 = code < 3;
  int a = ref1 ? code : code - 3;
  const real *size_ref = ref1 ? s1 : s2, *size_inc = ref1 ? s2 : s1, *pos_ref = ref1 ? g1.pos : g2.pos;
  const real* posoi = ref1 ? pos21 : pos12;
  const real* matref = ref1 ? g1.mat : g2.mat;
  real rinc[9];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) rinc[3 * i + j] = ref1 ? rot[3 * i + j] : rot[3 * j + i];
  real sign = posoi[a] >= 0.f ? 1.f : -1.f;
  int inc = 0;
  for (int k = 1; k < 3; ++k) if (r_abs(rinc[3 * a + k]) > r_abs(rinc[3 * a + inc])) inc = k;
  real incsign = sign * rinc[3 * a + inc] > 0.f ? -1.f : 1.f;
  int fx = (a + 1) % 3, fy = (a + 2) % 3, bu = (inc + 1) % 3, bv = (inc + 2) % 3;
  int coords[3] = {fx, fy, a};
  real cx[3], du[3], dv[3];
  for (int r = 0; r < 3; ++r) {
    int c = coords[r];
    cx[r] = posoi[c] + incsign * size_inc[inc] * rinc[3 * c + inc];
    du[r] = size_inc[bu] * rinc[3 * c + bu];
    dv[r] = size_inc[bv] * rinc[3 * c + bv];
  }
  cx[2] = sign * cx[2] - size_ref[a];
  du[2] *= sign;
  dv[2] *= sign;
  real poly[8][3];
  for (int k = 0; k < 4; ++k) {
    real su = (k == 0 || k == 3) ? 1.f : -1.f, sv = k < 2 ? 1.f : -1.f;
    for (int r = 0; r < 3; ++r) poly[k][r] = cx[r] + su * du[r] + sv * dv[r];
  }
  int count = 4;
  count = clip_face(count, poly, 0, 1.f, size_ref[fx]);
  count = clip_face(count, poly, 0, -1.f, size_ref[fx]);
  count = clip_face(count, poly, 1, 1.f, size_ref[fy]);
  count = clip_face(count, poly, 1, -1.f, size_ref[fy]);
  real n[3];
  axisf(matref, a, n);
  real ns = ref1 ? sign : -sign;
  n[0] *= ns; n[1] *= ns; n[2] *= ns;
  real duplicate = 1e-10f * (size_ref[fx] * size_ref[fx] + size_ref[fy] * size_ref[fy]);
  unsigned accepted = 0u;   // points kept so far (duplicates are tested against these only)
  for (int k = 0; k < count; ++k) {
    if (poly[k][2] > thr) continue;
    bool dupe = false;
    for (int q = 0; q < k; ++q) {
      if (!(accepted & (1u << q))) continue;
      real dx = poly[q][0] - poly[k][0], dy = poly[q][1] - poly[k][1];
      if (dx * dx + dy * dy < duplicate) { dupe = true; break; }
    }
    if (dupe) continue;
    accepted |= 1u << k;
    real local[3] = {0.f, 0.f, 0.f}, wpos[3];
    local[fx] = poly[k][0];
    local[fy] = poly[k][1];
    local[a] = sign * (size_ref[a] + 0.5f * poly[k][2]);
    mulmv3(matref, local, wpos);
    for (int r = 0; r < 3; ++r) wpos[r] += pos_ref[r];
    if (poly[k][2] < thr) raw_push(o, wpos, n, poly[k][2]);
  }
}

// Returns false for a type pair this build does not collide.  Inlined into the step's one
// out-of-line lane narrowphase, which builds both geoms in its own registers.
__device__ __forceinline__ bool narrowphase(KModel& m, const GeomX& __restrict__ g1, const GeomX& __restrict__ g2, real margin, RawOut& __restrict__ o) {
  o.n = 0;
  o.tangent_mask = 0u;
  int t1 = g1.type, t2 = g2.type;
  if (t1 == GT_PLANE) {
    if (t2 == GT_SPHERE) plane_point(g1, g2.pos, g2.size[0], margin, o);
    else if (t2 == GT_CAPSULE) plane_capsule(g1, g2, margin, o);
    else if (t2 == GT_BOX) plane_box(g1, g2, margin, o);
    else if (t2 == GT_MESH) plane_mesh(m, g1, g2, margin, o);
    return true;
  }
  if (t1 == GT_SPHERE && t2 == GT_SPHERE) {
    real fb[3] = {0.f, 0.f, 1.f};
    sphere_sphere(g1.pos, g1.size[0], g2.pos, g2.size[0], margin, o, fb);
    return true;
  }
  if (t1 == GT_SPHERE && t2 == GT_CAPSULE) {
    real a[3], b[3], s, t;
    segment_ends(g2, a, b);
    closest_segments(g1.pos, g1.pos, a, b, s, t);
    real p[3], fb[3] = {0.f, 0.f, 1.f};
    for (int k = 0; k < 3; ++k) p[k] = a[k] + (b[k] - a[k]) * t;
    sphere_sphere(g1.pos, g1.size[0], p, g2.size[0], margin, o, fb);
    return true;
  }
  if (t1 == GT_SPHERE && t2 == GT_BOX) { sphere_box(g1.pos, g1.size[0], g2, margin, o); return true; }
  if (t1 == GT_CAPSULE && t2 == GT_CAPSULE) { capsule_capsule(g1, g2, margin, o); return true; }
  if (t1 == GT_CAPSULE && t2 == GT_BOX) { capsule_box(g1, g2, margin, o); return true; }
  if (t1 == GT_BOX && t2 == GT_BOX) { box_box(g1, g2, margin, o); return true; }
  return false;
}

}  // namespace mx
