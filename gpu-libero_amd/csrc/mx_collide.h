// Narrowphase routines for the world-local kernel (FP32, one lane per candidate pair).
//
// Same geometric algorithms as the CPU oracle (oracle/oracle_collision.cpp), written for a single
// lane with register-resident state.  Reference leaves: plane-* gpu/cuda/collision/mjwarp_plane.cu:120-141,
// box-box SAT + face clipping mjwarp_box.cu:115-176 / mjwarp_box_manifold.cuh:105-133, capsule-box
// mjwarp_box.cu:33-102, sphere-box mjwarp_box.cu:14-32; capsule-capsule is new (MuJoCo semantics).
// Convention: the normal points from geom1 to geom2, pos is the midpoint between the surfaces,
// dist < 0 is penetration.
#pragma once
#include <hip/hip_runtime.h>
#include "mx_math.h"

namespace mx {

enum GeomType : int { GT_PLANE = 0, GT_SPHERE = 2, GT_CAPSULE = 3, GT_BOX = 6, GT_MESH = 7 };

constexpr int kMaxPairContacts = 4;

struct GeomX {
  int type;
  float pos[3], mat[9], size[3];
  const float* vert;   // mesh vertices (LDS), local frame
  int nvert;
};

struct RawOut {        // up to 4 contacts of one pair
  int n;
  float pos[kMaxPairContacts][3], normal[kMaxPairContacts][3], dist[kMaxPairContacts];
};

__device__ __forceinline__ float dot3f(const float* a, const float* b) { return a[0] * b[0] + a[1] * b[1] + a[2] * b[2]; }
__device__ __forceinline__ float norm3f(const float* a) { return sqrtf(dot3f(a, a)); }
__device__ __forceinline__ void axisf(const float* mat, int k, float* o) { o[0] = mat[k]; o[1] = mat[3 + k]; o[2] = mat[6 + k]; }
__device__ __forceinline__ void mulmtv3(const float* m, const float* v, float* r) {
  float a = m[0] * v[0] + m[3] * v[1] + m[6] * v[2];
  float b = m[1] * v[0] + m[4] * v[1] + m[7] * v[2];
  float c = m[2] * v[0] + m[5] * v[1] + m[8] * v[2];
  r[0] = a; r[1] = b; r[2] = c;
}

__device__ __forceinline__ void raw_push(RawOut& o, const float* pos, const float* n, float dist) {
  if (o.n >= kMaxPairContacts) return;
  for (int k = 0; k < 3; ++k) { o.pos[o.n][k] = pos[k]; o.normal[o.n][k] = n[k]; }
  o.dist[o.n] = dist;
  ++o.n;
}

// MJWarp make_frame: tangent from y (or z when the normal is close to y), then the cross product.
__device__ inline void make_frame(const float* n, float* frame) {
  float a[3] = {n[0], n[1], n[2]};
  float l = norm3f(a);
  if (l > 1e-15f) { a[0] /= l; a[1] /= l; a[2] /= l; }
  float b[3];
  if (-0.5f < a[1] && a[1] < 0.5f) { b[0] = 0.f; b[1] = 1.f; b[2] = 0.f; }
  else { b[0] = 0.f; b[1] = 0.f; b[2] = 1.f; }
  float d = dot3f(a, b);
  for (int k = 0; k < 3; ++k) b[k] -= a[k] * d;
  l = norm3f(b);
  if (l > 1e-15f) { b[0] /= l; b[1] /= l; b[2] /= l; }
  float c[3];
  cross3(a, b, c);
  for (int k = 0; k < 3; ++k) { frame[k] = a[k]; frame[3 + k] = b[k]; frame[6 + k] = c[k]; }
}

// ---------------------------------------------------------------- plane
__device__ inline void plane_point(const GeomX& p, const float* c, float r, float margin, RawOut& o) {
  float n[3];
  axisf(p.mat, 2, n);
  float d[3] = {c[0] - p.pos[0], c[1] - p.pos[1], c[2] - p.pos[2]};
  float dist = dot3f(n, d) - r;
  if (dist >= margin) return;
  float pos[3];
  for (int k = 0; k < 3; ++k) pos[k] = c[k] - n[k] * (r + 0.5f * dist);
  raw_push(o, pos, n, dist);
}

// Keep the 4 deepest vertices below the plane (ties by lower index), as the oracle.
__device__ inline void plane_vertices(const GeomX& p, const GeomX& g, float margin, RawOut& o) {
  float n[3];
  axisf(p.mat, 2, n);
  int nv = g.type == GT_BOX ? 8 : g.nvert;
  float bestd[4];
  int besti[4];
  int nb = 0;
  for (int i = 0; i < nv; ++i) {
    float l[3], v[3];
    if (g.type == GT_BOX) {
      l[0] = (i & 1) ? g.size[0] : -g.size[0];
      l[1] = (i & 2) ? g.size[1] : -g.size[1];
      l[2] = (i & 4) ? g.size[2] : -g.size[2];
    } else {
      l[0] = g.vert[3 * i]; l[1] = g.vert[3 * i + 1]; l[2] = g.vert[3 * i + 2];
    }
    mulmv3(g.mat, l, v);
    for (int k = 0; k < 3; ++k) v[k] += g.pos[k] - p.pos[k];
    float dist = dot3f(n, v);
    if (dist >= margin) continue;
    // insertion into the sorted best-4 list (stable: earlier index wins ties)
    int at = nb < 4 ? nb : 4;
    while (at > 0 && bestd[at - 1] > dist) --at;
    if (at >= 4) continue;
    int last = nb < 4 ? nb : 3;
    for (int q = last; q > at; --q) { bestd[q] = bestd[q - 1]; besti[q] = besti[q - 1]; }
    bestd[at] = dist;
    besti[at] = i;
    if (nb < 4) ++nb;
  }
  for (int q = 0; q < nb; ++q) {
    int i = besti[q];
    float l[3], v[3];
    if (g.type == GT_BOX) {
      l[0] = (i & 1) ? g.size[0] : -g.size[0];
      l[1] = (i & 2) ? g.size[1] : -g.size[1];
      l[2] = (i & 4) ? g.size[2] : -g.size[2];
    } else {
      l[0] = g.vert[3 * i]; l[1] = g.vert[3 * i + 1]; l[2] = g.vert[3 * i + 2];
    }
    mulmv3(g.mat, l, v);
    float pos[3];
    for (int k = 0; k < 3; ++k) pos[k] = g.pos[k] + v[k] - n[k] * 0.5f * bestd[q];
    raw_push(o, pos, n, bestd[q]);
  }
}

__device__ __forceinline__ void segment_ends(const GeomX& g, float* a, float* b) {
  float ax[3];
  axisf(g.mat, 2, ax);
  for (int k = 0; k < 3; ++k) { a[k] = g.pos[k] - g.size[1] * ax[k]; b[k] = g.pos[k] + g.size[1] * ax[k]; }
}

// ---------------------------------------------------------------- spheres and segments
__device__ inline void sphere_sphere(const float* c1, float r1, const float* c2, float r2, float margin,
                                     RawOut& o, const float* fallback) {
  float d[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
  float len = norm3f(d);
  float dist = len - r1 - r2;
  if (dist >= margin) return;
  float n[3];
  if (len > 1e-15f) { for (int k = 0; k < 3; ++k) n[k] = d[k] / len; }
  else { for (int k = 0; k < 3; ++k) n[k] = fallback[k]; }
  float pos[3];
  for (int k = 0; k < 3; ++k) pos[k] = c1[k] + n[k] * (r1 + 0.5f * dist);
  raw_push(o, pos, n, dist);
}

__device__ inline void closest_segments(const float* p1, const float* q1, const float* p2, const float* q2,
                                        float& s, float& t) {
  float d1[3], d2[3], r[3];
  for (int k = 0; k < 3; ++k) { d1[k] = q1[k] - p1[k]; d2[k] = q2[k] - p2[k]; r[k] = p1[k] - p2[k]; }
  float a = dot3f(d1, d1), e = dot3f(d2, d2), f = dot3f(d2, r);
  const float tiny = 1e-15f;
  if (a <= tiny && e <= tiny) { s = t = 0.f; return; }
  if (a <= tiny) { s = 0.f; t = fminf(fmaxf(f / e, 0.f), 1.f); return; }
  float c = dot3f(d1, r);
  if (e <= tiny) { t = 0.f; s = fminf(fmaxf(-c / a, 0.f), 1.f); return; }
  float b = dot3f(d1, d2), denom = a * e - b * b;
  s = denom > tiny * a * e ? fminf(fmaxf((b * f - c * e) / denom, 0.f), 1.f) : 0.f;
  t = (b * s + f) / e;
  if (t < 0.f) { t = 0.f; s = fminf(fmaxf(-c / a, 0.f), 1.f); }
  else if (t > 1.f) { t = 1.f; s = fminf(fmaxf((b - c) / a, 0.f), 1.f); }
}

__device__ inline void capsule_capsule(const GeomX& g1, const GeomX& g2, float margin, RawOut& o) {
  float a1[3], b1[3], a2[3], b2[3];
  segment_ends(g1, a1, b1);
  segment_ends(g2, a2, b2);
  float r1 = g1.size[0], r2 = g2.size[0];
  float d1[3], d2[3], cr[3];
  for (int k = 0; k < 3; ++k) { d1[k] = b1[k] - a1[k]; d2[k] = b2[k] - a2[k]; }
  cross3(d1, d2, cr);
  float l1 = norm3f(d1), l2 = norm3f(d2);
  float fb[3] = {cr[0], cr[1], cr[2]};
  float lf = norm3f(fb);
  if (lf < 1e-15f) { fb[0] = 0.f; fb[1] = 0.f; fb[2] = 1.f; }
  else { fb[0] /= lf; fb[1] /= lf; fb[2] /= lf; }
  if (l1 > 1e-15f && l2 > 1e-15f && norm3f(cr) < 1e-3f * l1 * l2) {
    float u[3] = {d1[0] / l1, d1[1] / l1, d1[2] / l1};
    float ta[3] = {a2[0] - a1[0], a2[1] - a1[1], a2[2] - a1[2]}, tb[3] = {b2[0] - a1[0], b2[1] - a1[1], b2[2] - a1[2]};
    float s0 = dot3f(ta, u), s1 = dot3f(tb, u);
    float lo = fmaxf(fminf(s0, s1), 0.f), hi = fminf(fmaxf(s0, s1), l1);
    if (hi - lo > 1e-6f * l1) {
      for (int e = 0; e < 2; ++e) {
        float sp = e == 0 ? lo : hi;
        float p1[3], p2[3];
        for (int k = 0; k < 3; ++k) p1[k] = a1[k] + u[k] * sp;
        float t = fminf(fmaxf((sp - s0) / (s1 - s0), 0.f), 1.f);
        for (int k = 0; k < 3; ++k) p2[k] = a2[k] + d2[k] * t;
        sphere_sphere(p1, r1, p2, r2, margin, o, fb);
      }
      return;
    }
  }
  float s, t;
  closest_segments(a1, b1, a2, b2, s, t);
  float p1[3], p2[3];
  for (int k = 0; k < 3; ++k) { p1[k] = a1[k] + d1[k] * s; p2[k] = a2[k] + d2[k] * t; }
  sphere_sphere(p1, r1, p2, r2, margin, o, fb);
}

// signed distance from p to box g and the outward normal at the closest surface point
__device__ inline float point_box(const GeomX& g, const float* p, float* normal) {
  float d[3] = {p[0] - g.pos[0], p[1] - g.pos[1], p[2] - g.pos[2]}, l[3];
  mulmtv3(g.mat, d, l);
  bool inside = true;
  float c[3];
  for (int k = 0; k < 3; ++k) {
    c[k] = fminf(fmaxf(l[k], -g.size[k]), g.size[k]);
    inside &= fabsf(l[k]) <= g.size[k];
  }
  if (!inside) {
    float diff[3] = {l[0] - c[0], l[1] - c[1], l[2] - c[2]};
    float len = norm3f(diff);
    float nl[3] = {diff[0] / len, diff[1] / len, diff[2] / len};
    mulmv3(g.mat, nl, normal);
    return len;
  }
  int best = 0;
  float gap = g.size[0] - fabsf(l[0]);
  for (int k = 1; k < 3; ++k)
    if (g.size[k] - fabsf(l[k]) < gap) { gap = g.size[k] - fabsf(l[k]); best = k; }
  float nl[3] = {0.f, 0.f, 0.f};
  nl[best] = l[best] >= 0.f ? 1.f : -1.f;
  mulmv3(g.mat, nl, normal);
  return -gap;
}

__device__ inline void sphere_box(const float* c, float r, const GeomX& box, float margin, RawOut& o) {
  float nb[3];
  float sd = point_box(box, c, nb);
  float dist = sd - r;
  if (dist >= margin) return;
  float n[3] = {-nb[0], -nb[1], -nb[2]}, pos[3];
  for (int k = 0; k < 3; ++k) pos[k] = c[k] + n[k] * (r + 0.5f * dist);
  raw_push(o, pos, n, dist);
}

__device__ inline void capsule_box(const GeomX& cap, const GeomX& box, float margin, RawOut& o) {
  float a[3], b[3];
  segment_ends(cap, a, b);
  float r = cap.size[0];
  RawOut ends;
  ends.n = 0;
  sphere_box(a, r, box, margin, ends);
  sphere_box(b, r, box, margin, ends);
  for (int q = 0; q < ends.n; ++q) raw_push(o, ends.pos[q], ends.normal[q], ends.dist[q]);
  if (ends.n == 2) return;
  float lo = 0.f, hi = 1.f;
  for (int it = 0; it < 40; ++it) {
    float m1 = lo + (hi - lo) / 3.f, m2 = hi - (hi - lo) / 3.f;
    float p1[3], p2[3], nn[3];
    for (int k = 0; k < 3; ++k) { p1[k] = a[k] + (b[k] - a[k]) * m1; p2[k] = a[k] + (b[k] - a[k]) * m2; }
    if (point_box(box, p1, nn) <= point_box(box, p2, nn)) hi = m2; else lo = m1;
  }
  float tm = 0.5f * (lo + hi);
  if (tm > 1e-3f && tm < 1.f - 1e-3f) {
    float pm[3];
    for (int k = 0; k < 3; ++k) pm[k] = a[k] + (b[k] - a[k]) * tm;
    sphere_box(pm, r, box, margin, o);
  }
}

// ---------------------------------------------------------------- box-box: SAT + face clipping
// Candidate points before reduction (at most 8 from clipping a quad by 4 planes).
struct Poly {
  int n;
  float p[8][3];
};

__device__ inline void clip_plane(Poly& poly, const float* n, float d) {
  Poly out;
  out.n = 0;
  for (int i = 0; i < poly.n; ++i) {
    const float* p = poly.p[i];
    const float* q = poly.p[(i + 1) % poly.n];
    float dp = n[0] * p[0] + n[1] * p[1] + n[2] * p[2] - d;
    float dq = n[0] * q[0] + n[1] * q[1] + n[2] * q[2] - d;
    if (dp <= 0.f && out.n < 8) { for (int k = 0; k < 3; ++k) out.p[out.n][k] = p[k]; ++out.n; }
    if (((dp < 0.f && dq > 0.f) || (dp > 0.f && dq < 0.f)) && out.n < 8) {
      float t = dp / (dp - dq);
      for (int k = 0; k < 3; ++k) out.p[out.n][k] = p[k] + (q[k] - p[k]) * t;
      ++out.n;
    }
  }
  poly = out;
}

// reduce candidate contacts to 4: deepest, farthest, largest triangle, largest added area
__device__ inline void reduce4_emit(const float (*pos)[3], const float* dist, int n, const float* normal, RawOut& o) {
  if (n <= 4) {
    for (int i = 0; i < n; ++i) raw_push(o, pos[i], normal, dist[i]);
    return;
  }
  unsigned used = 0;
  int i0 = 0;
  for (int i = 1; i < n; ++i) if (dist[i] < dist[i0]) i0 = i;
  used |= 1u << i0;
  int i1 = -1;
  float best = -1.f;
  for (int i = 0; i < n; ++i) {
    if (used & (1u << i)) continue;
    float d[3] = {pos[i][0] - pos[i0][0], pos[i][1] - pos[i0][1], pos[i][2] - pos[i0][2]};
    float v = dot3f(d, d);
    if (v > best) { best = v; i1 = i; }
  }
  used |= 1u << i1;
  int i2 = -1;
  best = -1.f;
  for (int i = 0; i < n; ++i) {
    if (used & (1u << i)) continue;
    float u[3], v[3], c[3];
    for (int k = 0; k < 3; ++k) { u[k] = pos[i1][k] - pos[i0][k]; v[k] = pos[i][k] - pos[i0][k]; }
    cross3(u, v, c);
    float a = dot3f(c, c);
    if (a > best) { best = a; i2 = i; }
  }
  used |= 1u << i2;
  int i3 = -1;
  best = -1.f;
  int tri[3] = {i0, i1, i2};
  for (int i = 0; i < n; ++i) {
    if (used & (1u << i)) continue;
    float add = 0.f;
    for (int e = 0; e < 3; ++e) {
      float u[3], v[3], c[3];
      for (int k = 0; k < 3; ++k) { u[k] = pos[tri[(e + 1) % 3]][k] - pos[tri[e]][k]; v[k] = pos[i][k] - pos[tri[e]][k]; }
      cross3(u, v, c);
      add = fmaxf(add, dot3f(c, c));
    }
    if (add > best) { best = add; i3 = i; }
  }
  int keep[4] = {i0, i1, i2, i3};
  for (int q = 0; q < 4; ++q) raw_push(o, pos[keep[q]], normal, dist[keep[q]]);
}

__device__ inline void face_contact(const GeomX& ref, int face, const float* nref, const GeomX& inc, float margin,
                                    bool flip, RawOut& o) {
  int best = 0;
  float bd = 0.f;
  for (int k = 0; k < 3; ++k) {
    float ax[3];
    axisf(inc.mat, k, ax);
    float d = dot3f(ax, nref);
    if (k == 0 || fabsf(d) > fabsf(bd)) { bd = d; best = k; }
  }
  float ninc[3];
  axisf(inc.mat, best, ninc);
  float sgn = bd > 0.f ? -1.f : 1.f;
  float u[3], v[3], ctr[3];
  int k1 = (best + 1) % 3, k2 = (best + 2) % 3;
  axisf(inc.mat, k1, u);
  axisf(inc.mat, k2, v);
  for (int k = 0; k < 3; ++k) ctr[k] = inc.pos[k] + sgn * ninc[k] * inc.size[best];
  Poly poly;
  poly.n = 4;
  const float su[4] = {1.f, -1.f, -1.f, 1.f}, sv[4] = {1.f, 1.f, -1.f, -1.f};
  for (int i = 0; i < 4; ++i)
    for (int k = 0; k < 3; ++k) poly.p[i][k] = ctr[k] + su[i] * inc.size[k1] * u[k] + sv[i] * inc.size[k2] * v[k];
  for (int j = 1; j <= 2; ++j) {
    int kk = (face + j) % 3;
    float ax[3];
    axisf(ref.mat, kk, ax);
    float c = dot3f(ax, ref.pos);
    clip_plane(poly, ax, c + ref.size[kk]);
    float nax[3] = {-ax[0], -ax[1], -ax[2]};
    clip_plane(poly, nax, -c + ref.size[kk]);
    if (poly.n == 0) return;
  }
  float off = dot3f(nref, ref.pos) + ref.size[face];
  float pos[8][3], dist[8];
  int n = 0;
  for (int i = 0; i < poly.n; ++i) {
    const float* q = poly.p[i];
    float sep = nref[0] * q[0] + nref[1] * q[1] + nref[2] * q[2] - off;
    if (sep >= margin) continue;
    for (int k = 0; k < 3; ++k) pos[n][k] = q[k] - nref[k] * 0.5f * sep;
    dist[n] = sep;
    ++n;
  }
  float normal[3] = {flip ? -nref[0] : nref[0], flip ? -nref[1] : nref[1], flip ? -nref[2] : nref[2]};
  reduce4_emit(pos, dist, n, normal, o);
}

__device__ inline void box_box(const GeomX& g1, const GeomX& g2, float margin, RawOut& o) {
  float A[3][3], B[3][3], d[3];
  for (int k = 0; k < 3; ++k) { axisf(g1.mat, k, A[k]); axisf(g2.mat, k, B[k]); d[k] = g2.pos[k] - g1.pos[k]; }
  float best_face = 1e30f, best_edge = 1e30f;
  int face_axis = -1, edge_i = -1, edge_j = -1;
  float face_n[3] = {0.f, 0.f, 0.f}, edge_n[3] = {0.f, 0.f, 0.f};
  for (int a = 0; a < 15; ++a) {
    float u[3];
    bool edge = a >= 6;
    int ei = 0, ej = 0;
    if (a < 3) { u[0] = A[a][0]; u[1] = A[a][1]; u[2] = A[a][2]; }
    else if (a < 6) { u[0] = B[a - 3][0]; u[1] = B[a - 3][1]; u[2] = B[a - 3][2]; }
    else {
      ei = (a - 6) / 3; ej = (a - 6) % 3;
      cross3(A[ei], B[ej], u);
      float len = norm3f(u);
      if (len < 1e-6f) continue;
      u[0] /= len; u[1] /= len; u[2] /= len;
    }
    float ra = 0.f, rb = 0.f;
    for (int k = 0; k < 3; ++k) { ra += g1.size[k] * fabsf(dot3f(u, A[k])); rb += g2.size[k] * fabsf(dot3f(u, B[k])); }
    float s = dot3f(u, d);
    float ov = ra + rb - fabsf(s);
    if (ov < -margin) return;
    float sg = s >= 0.f ? 1.f : -1.f;
    if (!edge) {
      if (ov < best_face) { best_face = ov; face_axis = a; for (int k = 0; k < 3; ++k) face_n[k] = sg * u[k]; }
    } else if (ov < best_edge) {
      best_edge = ov; edge_i = ei; edge_j = ej;
      for (int k = 0; k < 3; ++k) edge_n[k] = sg * u[k];
    }
  }
  if (edge_i >= 0 && best_edge < 0.95f * best_face - 1e-5f) {
    float c1[3], c2[3];
    for (int k = 0; k < 3; ++k) { c1[k] = g1.pos[k]; c2[k] = g2.pos[k]; }
    for (int k = 0; k < 3; ++k) {
      if (k != edge_i) {
        float s = dot3f(A[k], edge_n) >= 0.f ? 1.f : -1.f;
        for (int c = 0; c < 3; ++c) c1[c] += s * g1.size[k] * A[k][c];
      }
      if (k != edge_j) {
        float s = dot3f(B[k], edge_n) >= 0.f ? -1.f : 1.f;
        for (int c = 0; c < 3; ++c) c2[c] += s * g2.size[k] * B[k][c];
      }
    }
    float p1[3], q1[3], p2[3], q2[3];
    for (int c = 0; c < 3; ++c) {
      p1[c] = c1[c] - g1.size[edge_i] * A[edge_i][c]; q1[c] = c1[c] + g1.size[edge_i] * A[edge_i][c];
      p2[c] = c2[c] - g2.size[edge_j] * B[edge_j][c]; q2[c] = c2[c] + g2.size[edge_j] * B[edge_j][c];
    }
    float s, t;
    closest_segments(p1, q1, p2, q2, s, t);
    float pos[3];
    for (int c = 0; c < 3; ++c) pos[c] = 0.5f * (p1[c] + (q1[c] - p1[c]) * s + p2[c] + (q2[c] - p2[c]) * t);
    raw_push(o, pos, edge_n, -best_edge);
    return;
  }
  if (face_axis < 3) {
    face_contact(g1, face_axis, face_n, g2, margin, false, o);
  } else {
    float nref[3] = {-face_n[0], -face_n[1], -face_n[2]};
    face_contact(g2, face_axis - 3, nref, g1, margin, true, o);
  }
}

// Returns false for a type pair this build does not collide.
__device__ inline bool narrowphase(const GeomX& g1, const GeomX& g2, float margin, RawOut& o) {
  o.n = 0;
  int t1 = g1.type, t2 = g2.type;
  if (t1 == GT_PLANE) {
    if (t2 == GT_SPHERE) plane_point(g1, g2.pos, g2.size[0], margin, o);
    else if (t2 == GT_CAPSULE) {
      float a[3], b[3];
      segment_ends(g2, a, b);
      plane_point(g1, a, g2.size[0], margin, o);
      plane_point(g1, b, g2.size[0], margin, o);
    } else if (t2 == GT_BOX || t2 == GT_MESH) plane_vertices(g1, g2, margin, o);
    return true;
  }
  if (t1 == GT_SPHERE && t2 == GT_SPHERE) {
    float fb[3] = {0.f, 0.f, 1.f};
    sphere_sphere(g1.pos, g1.size[0], g2.pos, g2.size[0], margin, o, fb);
    return true;
  }
  if (t1 == GT_SPHERE && t2 == GT_CAPSULE) {
    float a[3], b[3], s, t;
    segment_ends(g2, a, b);
    closest_segments(g1.pos, g1.pos, a, b, s, t);
    float p[3], fb[3] = {0.f, 0.f, 1.f};
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
