// Convex narrowphase for the world-local kernel: GJK per lane, EPA cooperatively by the wave.
//
// Restates the reference's rigid CCD (FP32 as the reference):
//   support functions        gpu/cuda/collision/mjwarp_convex_geometry.cuh:17-68
//   signed-volume distance   gpu/cuda/collision/mjwarp_convex_simplex.cuh:13-79
//   GJK with cutoff          gpu/cuda/collision/mjwarp_convex_gjk.cuh:21-88
//   GJK phase and EPA        gpu/cuda/collision/mjwarp_convex_epa.cuh:18-261
//   box-box manifold         gpu/cuda/collision/mjwarp_box_manifold.cuh:7-133
//   pair driver              gpu/cuda/collision/mjwarp_convex_collision.cuh:43-79
// The reference runs one thread per candidate with the EPA polytope in a global scratch pool.
// Here each lane runs GJK for its candidate in registers; pairs that need EPA are then expanded one
// at a time by the whole wave, with the polytope in LDS (face argmin, visibility tests, horizon
// face attachment and repeated-vertex tests are lane-parallel; the order-dependent horizon edge
// list is built by lane 0 in face order, as the sequential algorithm does).  Hull support scans
// the hull's vertices (the reference hill-climbs the hull graph; both return the maximizer).
// Provenance: the routines restated here follow reference files headed "Copyright 2025 The Newton
// Developers, SPDX-License-Identifier: Apache-2.0" (MJWarp-derived CUDA in gpu/cuda/collision/);
// their feature selection, tolerances and step order are kept so that the contact sets match.  The
// MPR section restates libccd (BSD licence; its notice is reproduced there).
#pragma once
#include "mx_collide.h"

namespace MX_NS {
namespace cvx {

struct V {
  real v[3];
  __device__ real& operator[](int i) { return v[i]; }
  __device__ real operator[](int i) const { return v[i]; }
};
__device__ __forceinline__ V mk(real x, real y, real z) { V r; r.v[0] = x; r.v[1] = y; r.v[2] = z; return r; }
template <class P> __device__ __forceinline__ V ld(const P* p) { return mk(p[0], p[1], p[2]); }
template <class P> __device__ __forceinline__ void st(P* p, V a) { p[0] = a[0]; p[1] = a[1]; p[2] = a[2]; }
__device__ __forceinline__ V operator+(V a, V b) { return mk(a[0] + b[0], a[1] + b[1], a[2] + b[2]); }
__device__ __forceinline__ V operator-(V a, V b) { return mk(a[0] - b[0], a[1] - b[1], a[2] - b[2]); }
__device__ __forceinline__ V operator-(V a) { return mk(-a[0], -a[1], -a[2]); }
__device__ __forceinline__ V operator*(V a, real s) { return mk(a[0] * s, a[1] * s, a[2] * s); }
__device__ __forceinline__ V operator*(real s, V a) { return a * s; }
__device__ __forceinline__ real dot(V a, V b) { return a[0] * b[0] + a[1] * b[1] + a[2] * b[2]; }
__device__ __forceinline__ V crs(V a, V b) {
  return mk(a[1] * b[2] - a[2] * b[1], a[2] * b[0] - a[0] * b[2], a[0] * b[1] - a[1] * b[0]);
}
__device__ __forceinline__ V unit(V a) { real n = r_sqrt(dot(a, a)); return n > 0.f ? a * (1.0f / n) : mk(0.f, 0.f, 0.f); }
__device__ __forceinline__ V divv(V a, real s) { return mk(a[0] / s, a[1] / s, a[2] / s); }
template <class P> __device__ __forceinline__ V rot(const P* R, V x) {
  return mk(R[0] * x[0] + R[1] * x[1] + R[2] * x[2], R[3] * x[0] + R[4] * x[1] + R[5] * x[2],
            R[6] * x[0] + R[7] * x[1] + R[8] * x[2]);
}
template <class P> __device__ __forceinline__ V rotT(const P* R, V x) {
  return mk(R[0] * x[0] + R[3] * x[1] + R[6] * x[2], R[1] * x[0] + R[4] * x[1] + R[7] * x[2],
            R[2] * x[0] + R[5] * x[1] + R[8] * x[2]);
}
__device__ __forceinline__ real sgn(real x) { return x > 0.f ? 1.f : x < 0.f ? -1.f : 0.f; }

constexpr real kFloatMax = 1e30f, kConvexMin = 1e-15f;
constexpr real kAlign = 0.99605101346969604f, kPerp = 0.088782943785190582f;
constexpr int kHorizon = 24;

// ---------------------------------------------------------------- support
struct CGeom {
  V pos, size;
  const sreal* rot;   // world rotation (LDS)
  const sfloat* vert;  // hull vertices, geom frame (LDS), 4 floats per vertex
  int type, nvert, cached;
  real margin;
};
struct Support { V point; int cached, vertex; };

__device__ inline Support support(const CGeom& g, V d) {
  Support s{mk(0.f, 0.f, 0.f), -1, -1};
  if (g.type == GT_SPHERE) { s.point = g.pos + (g.size[0] + 0.5f * g.margin) * d; return s; }
  V local = rotT(g.rot, d), res = mk(0.f, 0.f, 0.f);
  if (g.type == GT_BOX) {
    V sign = mk(local[0] > 0.f ? 1.f : -1.f, local[1] > 0.f ? 1.f : -1.f, local[2] > 0.f ? 1.f : -1.f);
    for (int k = 0; k < 3; ++k) res[k] = sign[k] * g.size[k];
    s.point = rot(g.rot, res) + g.pos;
    s.vertex = int(sign[0] > 0.f) + 2 * int(sign[1] > 0.f) + 4 * int(sign[2] > 0.f);
  } else if (g.type == GT_CAPSULE) {
    res = local * g.size[0];
    res[2] += sgn(local[2]) * g.size[1];
    s.point = rot(g.rot, res) + g.pos;
  } else if (g.type == GT_MESH) {
    real best = -1e30f;
    if (g.cached > -1) { s.cached = g.cached; s.point = ld(g.vert + 4 * g.cached); best = dot(s.point, local); }
    // ascending scan, two vertices per round (their loads issue together)
    for (int i0 = 0; i0 < g.nvert; i0 += 2) {
      v4f q[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
        q[u] = *(const sfloat4*)(g.vert + 4 * (i0 + u < g.nvert ? i0 + u : i0));   // vertices padded to 16 bytes
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (i0 + u >= g.nvert) continue;
        V v = mk(q[u].x, q[u].y, q[u].z);
        real h = dot(v, local);
        if (h > best) { best = h; s.point = v; s.cached = i0 + u; }
      }
    }
    s.vertex = s.cached;
    s.point = rot(g.rot, s.point) + g.pos;
  }
  if (g.margin > 0.f) s.point = s.point + d * (0.5f * g.margin);
  return s;
}

// ---------------------------------------------------------------- signed-volume distance
struct W4 { real w[4]; };
__device__ __forceinline__ W4 w4(real a, real b, real c, real d) { W4 r; r.w[0] = a; r.w[1] = b; r.w[2] = c; r.w[3] = d; return r; }
__device__ __forceinline__ bool same_sign(real a, real b) { return (a > 0.f && b > 0.f) || (a < 0.f && b < 0.f); }

__device__ inline V origin_on_line(V a, V b) {
  V d = b - a;
  real s = -dot(b, d) / dot(d, d);
  return b + s * d;
}

__device__ inline V origin_on_plane(V a, V b, V c, bool& degenerate) {
  V d21 = b - a, d31 = c - a, d32 = c - b;
  degenerate = false;
  V n = crs(d32, d21);
  real nv = dot(n, b), nn = dot(n, n);
  if (nn == 0.f) { degenerate = true; return mk(0.f, 0.f, 0.f); }
  if (nv != 0.f && nn > kConvexMin) return (nv / nn) * n;
  n = crs(d21, d31);
  nv = dot(n, a); nn = dot(n, n);
  if (nn == 0.f) { degenerate = true; return mk(0.f, 0.f, 0.f); }
  if (nv != 0.f && nn > kConvexMin) return (nv / nn) * n;
  n = crs(d31, d32);
  nv = dot(n, c); nn = dot(n, n);
  return (nv / nn) * n;
}

// Component i of v by selects: a runtime index into the array would put v in scratch memory.
__device__ __forceinline__ real comp(V v, int i) { return i == 0 ? v[0] : (i == 1 ? v[1] : v[2]); }

__device__ inline W4 simplex1(V a, V b) {
  V p = origin_on_line(a, b);
  real mx = a[0] - b[0];
  int idx = 0;
  for (int k = 1; k < 3; ++k) { real v = a[k] - b[k]; if (r_abs(v) >= r_abs(mx)) { mx = v; idx = k; } }
  real c1 = comp(p, idx) - comp(b, idx), c2 = comp(a, idx) - comp(p, idx);
  if (same_sign(mx, c1) && same_sign(mx, c2)) return w4(c1 / mx, c2 / mx, 0.f, 0.f);
  return w4(0.f, 1.f, 0.f, 0.f);
}

__device__ __forceinline__ real minor2(V a, V b, V c, int i, int j) {
  V u = b - a, v = c - a;
  return comp(u, i) * comp(v, j) - comp(u, j) * comp(v, i);
}
__device__ __forceinline__ real area2(V p, V a, V b, int i, int j) {
  V u = a - p, v = b - p;
  return comp(u, i) * comp(v, j) - comp(u, j) * comp(v, i);
}

__device__ inline W4 simplex2(V a, V b, V c) {
  bool deg;
  V p = origin_on_plane(a, b, c, deg);
  if (deg) return simplex1(a, b);
  real m14 = minor2(a, b, c, 1, 2), m24 = minor2(a, b, c, 0, 2), m34 = minor2(a, b, c, 0, 1), mx;
  int i, j;
  if (r_abs(m14) >= r_abs(m24) && r_abs(m14) >= r_abs(m34)) { mx = m14; i = 1; j = 2; }
  else if (r_abs(m24) >= r_abs(m34)) { mx = m24; i = 0; j = 2; }
  else { mx = m34; i = 0; j = 1; }
  real c31 = area2(p, b, c, i, j), c32 = area2(p, c, a, i, j), c33 = area2(p, a, b, i, j);
  bool k1 = same_sign(mx, c31), k2 = same_sign(mx, c32), k3 = same_sign(mx, c33);
  if (k1 && k2 && k3) return w4(c31 / mx, c32 / mx, c33 / mx, 0.f);
  W4 w = w4(0.f, 0.f, 0.f, 0.f);
  real best = kFloatMax;
  if (!k1) { W4 s = simplex1(b, c); V x = s.w[0] * b + s.w[1] * c; w = w4(0.f, s.w[0], s.w[1], 0.f); best = dot(x, x); }
  if (!k2) {
    W4 s = simplex1(a, c); V x = s.w[0] * a + s.w[1] * c; real d = dot(x, x);
    if (d < best) { w = w4(s.w[0], 0.f, s.w[1], 0.f); best = d; }
  }
  if (!k3) {
    W4 s = simplex1(a, b); V x = s.w[0] * a + s.w[1] * b; real d = dot(x, x);
    if (d < best) w = w4(s.w[0], s.w[1], 0.f, 0.f);
  }
  return w;
}

__device__ __forceinline__ real det3(V a, V b, V c) { return dot(a, crs(b, c)); }

__device__ inline W4 simplex3(V a, V b, V c, V d) {
  real c41 = -det3(b, c, d), c42 = det3(a, c, d), c43 = -det3(a, b, d), c44 = det3(a, b, c);
  real det = c41 + c42 + c43 + c44;
  bool k1 = same_sign(det, c41), k2 = same_sign(det, c42), k3 = same_sign(det, c43), k4 = same_sign(det, c44);
  if (k1 && k2 && k3 && k4) return w4(c41 / det, c42 / det, c43 / det, c44 / det);
  W4 w = w4(0.f, 0.f, 0.f, 0.f);
  real best = kFloatMax;
  if (!k1) {
    W4 s = simplex2(b, c, d); V x = s.w[0] * b + s.w[1] * c + s.w[2] * d;
    w = w4(0.f, s.w[0], s.w[1], s.w[2]); best = dot(x, x);
  }
  if (!k2) {
    W4 s = simplex2(a, c, d); V x = s.w[0] * a + s.w[1] * c + s.w[2] * d; real e = dot(x, x);
    if (e < best) { w = w4(s.w[0], 0.f, s.w[1], s.w[2]); best = e; }
  }
  if (!k3) {
    W4 s = simplex2(a, b, d); V x = s.w[0] * a + s.w[1] * b + s.w[2] * d; real e = dot(x, x);
    if (e < best) { w = w4(s.w[0], s.w[1], 0.f, s.w[2]); best = e; }
  }
  if (!k4) {
    W4 s = simplex2(a, b, c); V x = s.w[0] * a + s.w[1] * b + s.w[2] * c; real e = dot(x, x);
    if (e < best) w = w4(s.w[0], s.w[1], s.w[2], 0.f);
  }
  return w;
}

// ---------------------------------------------------------------- GJK
struct Gjk {
  bool separated;
  real dist;
  V x1, x2;
  int dim;
  V s[4], s1[4], s2[4];
  int v1[4], v2[4], index1, index2;
};

__device__ inline Gjk gjk(real tol, int maxit, CGeom g1, CGeom g2, V init1, V init2, real cutoff, bool discrete) {
  // The simplex lives in registers: every access below uses compile-time slot indices (slot
  // writes and the compaction after the distance sub-algorithm are unrolled selects).
  Gjk r;
#pragma unroll
  for (int k = 0; k < 4; ++k) { r.s[k] = r.s1[k] = r.s2[k] = mk(0.f, 0.f, 0.f); r.v1[k] = r.v2[k] = 0; }
  int n = 0;
  W4 w = w4(1.f, 0.f, 0.f, 0.f);
  real eps = discrete ? 0.f : 0.5f * tol * tol, min_norm = discrete ? kConvexMin : tol;
  V x = init1 - init2;
  real norm = r_sqrt(dot(x, x)), prev = 0.f;
  for (int it = 0; it < maxit; ++it) {
    if (norm < min_norm || r_abs(prev - norm) < kConvexMin) break;
    V dir = divv(x, norm);
    if (discrete && norm < 1e-4f) {
      if (n == 2) {
        V e = r.s[1] - r.s[0];
        real l2 = dot(e, e);
        if (l2 > 1e-30f) {
          dir = dir - (dot(dir, e) / l2) * e;
          real l = r_sqrt(dot(dir, dir));
          if (l > kConvexMin) dir = divv(dir, l);
        }
      } else if (n == 3) {
        V nn = crs(r.s[1] - r.s[0], r.s[2] - r.s[0]);
        real l = r_sqrt(dot(nn, nn));
        if (l > kConvexMin) dir = divv(sgn(dot(dir, nn)) * nn, l);
      }
    }
    Support a = support(g1, -dir), b = support(g2, dir);
    g1.cached = a.cached;
    g2.cached = b.cached;
    V sn = a.point - b.point;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k == n) { r.s1[k] = a.point; r.v1[k] = a.vertex; r.v2[k] = b.vertex; r.s[k] = sn; }
    if (dot(x, x - sn) < eps) break;
    real lower = dot(x, sn);
    bool cut = (cutoff == 0.f && lower > 0.f) || (cutoff != 0.f && cutoff < kFloatMax && lower > 0.f && lower >= cutoff * norm);
    if (cut && discrete && norm < 1e-4f && (n == 2 || n == 3)) {
      lower = dot(dir, sn);
      real cn = r_sqrt(dot(dir, dir));
      cut = cn > kConvexMin && lower > 0.f && (cutoff == 0.f || (cutoff < kFloatMax && lower >= cutoff * cn));
    }
    if (cut) {
      r.separated = true; r.dim = 0; r.dist = kFloatMax; r.index1 = g1.cached; r.index2 = g2.cached;
      r.x1 = r.x2 = mk(0.f, 0.f, 0.f);
      return r;
    }
    int cnt = n + 1;
    if (cnt == 4) w = simplex3(r.s[0], r.s[1], r.s[2], r.s[3]);
    else if (cnt == 3) w = simplex2(r.s[0], r.s[1], r.s[2]);
    else if (cnt == 2) w = simplex1(r.s[0], r.s[1]);
    else w = w4(1.f, 0.f, 0.f, 0.f);
    // keep the vertices with nonzero weight, in order: compacted in place (slot n <= i, so no
    // slot is overwritten before it is read)
    n = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (w.w[i] == 0.f) continue;
#pragma unroll
      for (int j = 0; j < i; ++j)
        if (j == n) {
          r.s[j] = r.s[i]; r.s1[j] = r.s1[i]; r.v1[j] = r.v1[i]; r.v2[j] = r.v2[i];
          w.w[j] = w.w[i];
        }
      ++n;
    }
    if (n < 1) break;
    x = mk(0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < n) x = x + w.w[k] * r.s[k];
    prev = norm;
    norm = r_sqrt(dot(x, x));
    if (n == 4) break;
  }
  r.separated = false;
  // the support points on geom 2 are not carried through the loop (register pressure): s2 = s1 - s
#pragma unroll
  for (int k = 0; k < 4; ++k) r.s2[k] = r.s1[k] - r.s[k];
  if (n == 0) { r.x1 = init1; r.x2 = init2; }
  else {
    r.x1 = r.x2 = mk(0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < n) { r.x1 = r.x1 + w.w[k] * r.s1[k]; r.x2 = r.x2 + w.w[k] * r.s2[k]; }
  }
  if (norm > 0.f) {
    V dir = divv(x, norm);
    Support a = support(g1, -dir), b = support(g2, dir);
    r.separated = dot(x, a.point - b.point) > 0.f;
  }
  r.dist = n == 4 && !r.separated ? 0.f : norm;
  r.dim = n;
  r.index1 = g1.cached; r.index2 = g2.cached;
  return r;
}

__device__ __forceinline__ bool discrete_pair(int a, int b) {
  return (a == GT_BOX || a == GT_MESH) && (b == GT_BOX || b == GT_MESH);
}

struct Phase {
  bool needs_epa, require_enclosing;
  real distance;
  V x1, x2;
  Gjk r;
  int cached1, cached2;
};

__device__ inline Phase gjk_phase(real tol, real cutoff, int iters, CGeom a, CGeom b) {
  Phase ph;
  ph.needs_epa = false; ph.require_enclosing = false;
  V size1 = a.size, size2 = b.size;
  real m1 = a.margin, m2 = b.margin, full1 = 0.f, full2 = 0.f, r1 = 0.f, r2 = 0.f;
  bool discrete = discrete_pair(a.type, b.type) && m1 == 0.f && m2 == 0.f;
  if (a.type == GT_SPHERE || a.type == GT_CAPSULE) { r1 = a.size[0]; full1 = r1 + 0.5f * m1; a.margin = 0.f; a.size[0] = 0.f; }
  if (b.type == GT_SPHERE || b.type == GT_CAPSULE) { r2 = b.size[0]; full2 = r2 + 0.5f * m2; b.margin = 0.f; b.size[0] = 0.f; }
  if (r1 + r2 > 0.f) {
    cutoff += full1 + full2;
    Gjk r = gjk(tol, iters, a, b, a.pos, b.pos, cutoff, discrete);
    a.cached = r.index1; b.cached = r.index2;
    if (r.dist > tol) {
      ph.cached1 = a.cached; ph.cached2 = b.cached;
      if (r.dist == kFloatMax) { ph.distance = r.dist; ph.x1 = r.x1; ph.x2 = r.x2; return ph; }
      V n = unit(r.x2 - r.x1);
      ph.x1 = r.x1; ph.x2 = r.x2;
      if (full1 > 0.f) ph.x1 = ph.x1 + full1 * n;
      if (full2 > 0.f) ph.x2 = ph.x2 - full2 * n;
      ph.distance = r.dist - (full1 + full2);
      return ph;
    }
    a.size = size1; a.margin = m1; b.size = size2; b.margin = m2;
    cutoff -= full1 + full2;
  }
  Gjk r = gjk(tol, iters, a, b, a.pos, b.pos, cutoff, discrete);
  a.cached = r.index1; b.cached = r.index2;
  bool retry_box = a.type == GT_BOX && b.type == GT_BOX && discrete && r.dist > tol && r.dim >= 2 && !r.separated;
  if (retry_box) {
    Gjk q = gjk(tol, iters, a, b, r.x1, r.x2, cutoff, discrete);
    if (q.separated || (q.dim >= 2 && q.dist < r.dist)) r = q;
    a.cached = r.index1; b.cached = r.index2;
  }
  ph.cached1 = a.cached; ph.cached2 = b.cached;
  ph.distance = r.dist; ph.x1 = r.x1; ph.x2 = r.x2;
  if ((r.dist > tol && !retry_box) || r.dim < 2 || r.separated) return ph;
  ph.needs_epa = true;
  ph.require_enclosing = retry_box;
  ph.r = r;
  return ph;
}

// ---------------------------------------------------------------- EPA (wave-cooperative)
// LDS block of the one EPA in flight; `vc`, `fc` are the vertex and face capacities.
struct Poly {
  // always in LDS: aliasing the constraint rows on the LDS route, in the world's LDS window on the
  // workspace route
  sreal* vert;    // 2 * vc * 3: support point on geom 1, on geom 2
  sint* vidx;      // 2 * vc
  sint* face;      // fc packed a | b << 10 | c << 20; bit 31 deleted, bit 30 invalid
  sreal* proj;    // 3 * fc
  sreal* norm2;   // fc
  sint* sc;        // scalars (below)
  sreal* center;  // 3
  int vc, fc;
  __device__ V vertex(int i) const { return ld(vert + 6 * i) - ld(vert + 6 * i + 3); }
};
enum { P_NVERT, P_NFACE, P_NHOR, P_STATUS, P_INDEX, P_NVALID, P_STOP, P_NSC = 8 };

__host__ __device__ inline int poly_words(int vc, int fc) {
  return 6 * vc + 2 * vc + fc + 3 * fc + fc + P_NSC + 4;
}

__device__ inline Poly poly_at(sreal* base, int vc, int fc) {
  Poly p;
  int at = 0;
  p.vert = base + at; at += 6 * vc;
  p.vidx = (sint*)(base + at); at += 2 * vc;
  p.face = (sint*)(base + at); at += fc;
  p.proj = base + at; at += 3 * fc;
  p.norm2 = base + at; at += fc;
  p.sc = (sint*)(base + at); at += P_NSC;
  p.center = base + at;
  p.vc = vc; p.fc = fc;
  return p;
}

// The following run on one lane (the caller guards) unless stated.
__device__ inline real attach_face(Poly& p, int nface, int index, int a, int b, int c) {
  if (index >= p.fc || nface == p.fc) return 0.f;
  V one = p.vertex(a), two = p.vertex(b), three = p.vertex(c);
  bool bad;
  V r = origin_on_plane(three, two, one, bad);
  if (bad) return 0.f;
  if (dot(r, one - ld(p.center)) < 0.f) r = -r;
  p.face[index] = a + (b << 10) + (c << 20);
  st(p.proj + 3 * index, r);
  p.norm2[index] = dot(r, r);
  return p.norm2[index];
}

__device__ inline void poly_support(Poly& p, int index, const CGeom& a, const CGeom& b, V d, int& c1, int& c2) {
  Support one = support(a, d), two = support(b, -d);
  st(p.vert + 6 * index, one.point); st(p.vert + 6 * index + 3, two.point);
  p.vidx[2 * index] = one.vertex; p.vidx[2 * index + 1] = two.vertex;
  c1 = one.cached; c2 = two.cached;
}

__device__ inline void initial_vertices(Poly& p, const Gjk& r, int n) {
  for (int i = 0; i < n; ++i) {
    st(p.vert + 6 * i, r.s1[i]); st(p.vert + 6 * i + 3, r.s2[i]);
    p.vidx[2 * i] = r.v1[i]; p.vidx[2 * i + 1] = r.v2[i];
  }
}

__device__ inline void replace_triangle(const Poly& p, Gjk& r, int a, int b, int c) {
  int idx[3] = {a, b, c};
  for (int i = 0; i < 3; ++i) {
    int j = idx[i];
    r.s1[i] = ld(p.vert + 6 * j); r.s2[i] = ld(p.vert + 6 * j + 3); r.s[i] = r.s1[i] - r.s2[i];
    r.v1[i] = p.vidx[2 * j]; r.v2[i] = p.vidx[2 * j + 1];
  }
  r.dim = 3;
}

__device__ __forceinline__ bool same_side(V a, V b, V c, V d) {
  V n = crs(b - a, c - a);
  real one = dot(n, d - a), two = dot(n, -a);
  return (one > 0.f && two > 0.f) || (one < 0.f && two < 0.f);
}
__device__ __forceinline__ bool tetra_contains_origin(V a, V b, V c, V d) {
  return same_side(a, b, c, d) && same_side(b, c, d, a) && same_side(c, d, a, b) && same_side(d, a, b, c);
}

__device__ inline V triangle_affine(V a, V b, V c, V pt) {
  real m14 = minor2(a, b, c, 1, 2), m24 = minor2(a, b, c, 0, 2), m34 = minor2(a, b, c, 0, 1), mx;
  int i, j;
  if (r_abs(m14) >= r_abs(m24) && r_abs(m14) >= r_abs(m34)) { mx = m14; i = 1; j = 2; }
  else if (r_abs(m24) >= r_abs(m34)) { mx = m24; i = 0; j = 2; }
  else { mx = m34; i = 0; j = 1; }
  return mk(area2(pt, b, c, i, j) / mx, area2(pt, c, a, i, j) / mx, area2(pt, a, b, i, j) / mx);
}

__device__ inline bool triangle_contains(V a, V b, V c, V pt) {
  V w = triangle_affine(a, b, c, pt);
  if (w[0] < 0.f || w[1] < 0.f || w[2] < 0.f) return false;
  V d = w[0] * a + w[1] * b + w[2] * c - pt;
  return r_sqrt(dot(d, d)) < kConvexMin;
}

// Initial polytope around the GJK simplex (one lane).  Returns the status (0: ready).
__device__ inline int build_polytope(Poly& p, Gjk& r, const CGeom& a, const CGeom& b, bool& require_enclosing) {
  int nvert = 0, nface = 0, status = 0;
  int c1, c2;
  if (r.dim == 2) {
    V diff = r.s[1] - r.s[0];
    st(p.center, 0.5f * (r.s[0] + r.s[1]));
    int index = 0;
    real value = kFloatMax;
    for (int i = 0; i < 3; ++i) if (r_abs(diff[i]) < value) { value = r_abs(diff[i]); index = i; }
    V ax = mk(0.f, 0.f, 0.f);
    ax[index] = 1.f;
    V d1 = crs(ax, diff), u = divv(diff, r_sqrt(dot(diff, diff)));
    const real s3 = 0.86602540378f;
    real R[9];
    for (int i = 0; i < 3; ++i) for (int j = 0; j < 3; ++j) R[3 * i + j] = (i == j ? -0.5f : 0.f) + 1.5f * u[i] * u[j];
    R[1] -= u[2] * s3; R[2] += u[1] * s3; R[3] += u[2] * s3; R[5] -= u[0] * s3; R[6] -= u[1] * s3; R[7] += u[0] * s3;
    V dirs[3];
    dirs[0] = d1; dirs[1] = rot(R, d1); dirs[2] = rot(R, dirs[1]);
    initial_vertices(p, r, 2);
    for (int i = 0; i < 3; ++i) poly_support(p, i + 2, a, b, divv(dirs[i], r_sqrt(dot(dirs[i], dirs[i]))), c1, c2);
    const int faces[6][3] = {{0, 2, 3}, {0, 4, 2}, {0, 3, 4}, {1, 3, 2}, {1, 2, 4}, {1, 4, 3}};
    status = 0;
    for (int i = 0; i < 6; ++i)
      if (attach_face(p, 0, i, faces[i][0], faces[i][1], faces[i][2]) < 1e-10f) {
        status = -1;
        replace_triangle(p, r, faces[i][0], faces[i][1], faces[i][2]);
        break;
      }
    if (status == 0) {
      V v2 = p.vertex(2), v3 = p.vertex(3), v4 = p.vertex(4), v1 = r.s[0], base = r.s[1] - v1;
      real one = det3(v2 - v1, v3 - v1, base), two = det3(v3 - v1, v4 - v1, base), three = det3(v4 - v1, v2 - v1, base);
      if (!((one >= 0.f && two >= 0.f && three >= 0.f) || (one <= 0.f && two <= 0.f && three <= 0.f))) status = 1;
      else { nvert = 5; nface = 6; }
    }
  } else if (r.dim == 4) {
    st(p.center, 0.25f * (r.s[0] + r.s[1] + r.s[2] + r.s[3]));
    initial_vertices(p, r, 4);
    real dist[4];
    int closest = 0;
    const int faces[4][3] = {{0, 1, 2}, {0, 3, 1}, {0, 2, 3}, {3, 2, 1}};
    status = 0;
    for (int i = 0; i < 4; ++i) {
      dist[i] = attach_face(p, 0, i, faces[i][0], faces[i][1], faces[i][2]);
      if (dist[i] < 1e-17f) { status = -1; replace_triangle(p, r, faces[i][0], faces[i][1], faces[i][2]); break; }
      if (i == 1) closest = dist[0] < dist[1] ? 0 : 1;
      else if (i > 1 && dist[i] < dist[closest]) closest = i;
    }
    if (status == 0) {
      if (!tetra_contains_origin(r.s[0], r.s[1], r.s[2], r.s[3])) {
        if (dist[closest] > kConvexMin) status = 12;
        else { status = -1; replace_triangle(p, r, faces[closest][0], faces[closest][1], faces[closest][2]); }
      } else { nvert = 4; nface = 4; }
    }
  }
  if (r.dim == 3) {
    st(p.center, (r.s[0] + r.s[1] + r.s[2]) * (1.0f / 3.0f));
    V n = crs(r.s[1] - r.s[0], r.s[2] - r.s[0]);
    real norm = r_sqrt(dot(n, n));
    nvert = nface = 0;
    if (norm < kConvexMin) status = 2;
    else {
      n = divv(n, norm);
      initial_vertices(p, r, 3);
      poly_support(p, 3, a, b, -n, c1, c2);
      poly_support(p, 4, a, b, n, c1, c2);
      V v1 = r.s[0], v2 = r.s[1], v3 = r.s[2], v4 = p.vertex(3), v5 = p.vertex(4);
      if (triangle_contains(v1, v2, v3, v4)) status = 3;
      else if (triangle_contains(v1, v2, v3, v5)) status = 4;
      else if (r.dist > 1e-5f && !tetra_contains_origin(v1, v2, v3, v4) && !tetra_contains_origin(v1, v2, v3, v5)) status = 5;
      else {
        const int faces[6][3] = {{4, 0, 1}, {4, 2, 0}, {4, 1, 2}, {3, 1, 0}, {3, 0, 2}, {3, 2, 1}};
        bool box = a.type == GT_BOX && b.type == GT_BOX && a.margin == 0.f && b.margin == 0.f;
        status = 0;
        for (int i = 0; i < 6; ++i) {
          real d2 = attach_face(p, 0, i, faces[i][0], faces[i][1], faces[i][2]);
          if (require_enclosing || box) {
            if (!(d2 > 0.f)) { status = 6 + i; break; }
            if (d2 < 1e-10f) require_enclosing = true;
          } else if (d2 < 1e-10f) { status = 6 + i; break; }
        }
        if (status == 0) { nvert = 5; nface = 6; }
      }
    }
  }
  p.sc[P_NVERT] = nvert;
  p.sc[P_NFACE] = nface;
  p.sc[P_NHOR] = 0;
  p.sc[P_STATUS] = status;
  return status;
}

// half-space signs of every face with respect to the centre, in FP64 (one lane)
__device__ inline bool encloses_origin(const Poly& p) {
  int nvert = p.sc[P_NVERT], nface = p.sc[P_NFACE];
  if (nvert < 4 || nface < 4) return false;
  for (int i = 0; i < nface; ++i) {
    int f = p.face[i];
    V a = p.vertex(f & 1023), b = p.vertex((f >> 10) & 1023), c = p.vertex((f >> 20) & 1023);
    double u[3], v[3], n[3];
    for (int k = 0; k < 3; ++k) { u[k] = double(b[k]) - double(a[k]); v[k] = double(c[k]) - double(a[k]); }
    n[0] = u[1] * v[2] - u[2] * v[1]; n[1] = u[2] * v[0] - u[0] * v[2]; n[2] = u[0] * v[1] - u[1] * v[0];
    double origin = 0.0, center = 0.0;
    for (int k = 0; k < 3; ++k) { origin -= n[k] * double(a[k]); center += n[k] * (double(p.center[k]) - double(a[k])); }
    if (center == 0.0 || (origin > 0.0 && center < 0.0) || (origin < 0.0 && center > 0.0)) return false;
  }
  return true;
}

__device__ __forceinline__ bool face_deleted(int f) { return (unsigned(f) & 0x80000000u) != 0u; }
__device__ __forceinline__ bool face_invalid(int f) { return (unsigned(f) & 0xc0000000u) != 0u; }
__device__ __forceinline__ int face_mark(int f, unsigned bit) { return int(unsigned(f) | bit); }

// horizon_overflow: the horizon edge list exceeded kHorizon edges; the pair gives no contact and
// the world is flagged MX_OVERFLOW_EPA_HORIZON (the reference's epa_horizon_overflow,
// mjwarp_convex_epa.cuh:186-214).  redo: a small polytope (RowGroup) ran out of room; the pair is
// expanded again from the start on the wave's full-size polytope, which gives the same result.
struct EpaOut { real distance; int ncontact; V x1, x2; int face; bool horizon_overflow, redo; };

// The lanes that expand one polytope together.  WaveGroup: the whole wave, one polytope of the
// full capacity at a time.  RowGroup: one 16-lane row of the wave, so four polytopes expand at
// once; the polytope is small, and running out of its room (vertices, faces, or more horizon
// edges than the row has lanes) ends the expansion with `redo`.  Reductions are uniform over the
// group; ballot returns the group's lanes as bits 0..kSize-1.
struct WaveGroup {
  static constexpr int kSize = 64;
  static constexpr bool kSmall = false;
  int lane;
  __device__ explicit WaveGroup(int l) : lane(l) {}
  __device__ real min(real v) const { return wave_min(v); }
  __device__ int min(int v) const { return wave_min(v); }
  __device__ real max(real v) const { return wave_max(v); }
  __device__ unsigned long long ballot(bool p) const { return __ballot(p); }
  __device__ int read(int v, int j) const { return __builtin_amdgcn_readlane(v, j); }   // j uniform
  __device__ void fence() const { __syncthreads(); }
};
struct RowGroup {
  static constexpr int kSize = 16;
  static constexpr bool kSmall = true;
  int lane, base;
  __device__ explicit RowGroup(int l) : lane(l & 15), base(l & 48) {}
  __device__ real min(real v) const { return row_min(v); }
  __device__ int min(int v) const { return row_min(v); }
  __device__ real max(real v) const { return row_max(v); }
  __device__ unsigned long long ballot(bool p) const { return (__ballot(p) >> base) & 0xffffull; }
  __device__ int read(int v, int j) const { return __shfl(v, j, 16); }
  // the rows run different polytopes under different branches, so no barrier: LDS operations of
  // one wave complete in issue order, and the fence keeps the compiler from moving them across
  __device__ void fence() const {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }
};

// Support of a geom computed by the group's lanes (same result on every lane of the group).  Hull
// vertices are scanned in parallel; the sequential scan's choice is kept: the cached vertex unless
// another vertex is strictly higher, else the lowest index among the highest.
template <class G>
__device__ inline Support support_group(const CGeom& g, V d, const G& grp) {
  if (g.type != GT_MESH) return support(g, d);
  V local = rotT(g.rot, d);
  real best = -1e30f;
  int bi = -1;
  for (int i = grp.lane; i < g.nvert; i += G::kSize) {
    v4f q = *(const sfloat4*)(g.vert + 4 * i);
    real h = q.x * local[0] + q.y * local[1] + q.z * local[2];
    if (h > best) { best = h; bi = i; }
  }
  const real gmax = grp.max(best);
  const int mine = grp.min((bi >= 0 && best == gmax) ? bi : g.nvert);
  int pick = mine < g.nvert ? mine : 0;   // no comparable vertex (NaN direction): vertex 0
  Support s{mk(0.f, 0.f, 0.f), -1, -1};
  if (g.cached > -1) {
    v4f q = *(const sfloat4*)(g.vert + 4 * g.cached);
    real hc = q.x * local[0] + q.y * local[1] + q.z * local[2];
    if (!(gmax > hc)) pick = g.cached;
  }
  v4f q = *(const sfloat4*)(g.vert + 4 * pick);
  s.cached = pick;
  s.vertex = pick;
  s.point = rot(g.rot, mk(q.x, q.y, q.z)) + g.pos;
  if (g.margin > 0.f) s.point = s.point + d * (0.5f * g.margin);
  return s;
}

// Polytope expansion by a group of lanes (every lane of the group calls it with the same
// arguments).  The horizon edge list is held one edge per lane (lane i holds edge i), so the
// order-dependent insert / swap-remove of the sequential algorithm costs a ballot per edge.
template <class G>
__device__ inline EpaOut epa_expand(Poly& p, real tol, int iters, CGeom a, CGeom b, bool discrete, const G& g) {
  real upper = kFloatMax, upper2 = kFloatMax, eps = discrete ? 1e-7f : tol;
  int index = -1;
  int nface = p.sc[P_NFACE], nvert = p.sc[P_NVERT], nvalid = nface;
  bool horizon_overflow = false, redo = false;
  const int hcap = G::kSmall ? G::kSize : kHorizon;
  iters = min(iters, 1000);
  for (int it = 0; it < iters; ++it) {
    int prev = index;
    // face with the smallest distance to the origin (lowest index on ties)
    real best = kFloatMax;
    int bi = -1;
    for (int i = g.lane; i < nface; i += G::kSize)
      if (!face_invalid(p.face[i]) && p.norm2[i] < best) { best = p.norm2[i]; bi = i; }
    const real lower2 = g.min(best);
    const int low = g.min((bi >= 0 && best == lower2) ? bi : 0x7fffffff);
    index = low == 0x7fffffff ? -1 : low;
    if (lower2 > upper2 || index < 0) { index = prev; break; }
    if (lower2 <= 0.f) break;
    real lower = r_sqrt(lower2);
    int wi = nvert;
    V pr = ld(p.proj + 3 * index), dir = divv(pr, lower);
    Support one = support_group(a, dir, g), two = support_group(b, -dir, g);
    a.cached = one.cached;
    b.cached = two.cached;
    if (G::kSmall && wi >= p.vc) { redo = true; break; }
    if (g.lane == 0) {
      st(p.vert + 6 * wi, one.point); st(p.vert + 6 * wi + 3, two.point);
      p.vidx[2 * wi] = one.vertex; p.vidx[2 * wi + 1] = two.vertex;
    }
    ++nvert;
    V w = one.point - two.point;
    real next = dot(pr, w) / lower;
    if (next < upper) { upper = next; upper2 = upper * upper; }
    if (upper - lower < eps) break;
    if (discrete) {
      bool rep = false;
      for (int i = g.lane; i < wi; i += G::kSize) rep |= p.vidx[2 * i] == one.vertex && p.vidx[2 * i + 1] == two.vertex;
      if (g.ballot(rep)) break;
    }
    // horizon: remove the selected face, then every live face the new vertex sees, in face order
    int hreg = 0, nh = 0;
    bool overflow = false;
    auto add_edge = [&](int ea, int eb) {
      if (overflow) return;
      int edge = (min(ea, eb) << 10) | max(ea, eb);
      unsigned long long hit = g.ballot(g.lane < nh && hreg == edge);
      if (hit) {
        int j = __ffsll((long long)hit) - 1;
        int last = g.read(hreg, nh - 1);
        if (g.lane == j) hreg = last;
        --nh;
      } else if (nh == hcap) {
        overflow = true;
      } else {
        if (g.lane == nh) hreg = edge;
        ++nh;
      }
    };
    auto remove_face = [&](int i) {
      int f = p.face[i];
      g.fence();
      if (g.lane == 0) p.face[i] = face_mark(f, 0x80000000u);
      add_edge(f & 0x3ff, (f >> 10) & 0x3ff);
      add_edge((f >> 10) & 0x3ff, (f >> 20) & 0x3ff);
      add_edge((f >> 20) & 0x3ff, f & 0x3ff);
    };
    --nvalid;
    remove_face(index);
    for (int base = 0; base < nface && !overflow; base += G::kSize) {
      int i = base + g.lane;
      bool vis = false;
      if (i < nface && i != index && !face_deleted(p.face[i]))
        vis = dot(ld(p.proj + 3 * i), w) - p.norm2[i] > 1e-10f;
      unsigned long long mask = g.ballot(vis);
      while (mask && !overflow) {
        int k = base + __ffsll((long long)mask) - 1;
        mask &= mask - 1;
        if (!face_invalid(p.face[k])) --nvalid;
        remove_face(k);
      }
    }
    if (overflow) {
      index = -1;
      if (G::kSmall) redo = true;
      else horizon_overflow = true;
      break;
    }
    g.fence();
    if (G::kSmall && nface + nh > p.fc) { redo = true; break; }
    // one new face per horizon edge, in horizon order; stop at the first degenerate one
    real d2 = 1.f;
    if (g.lane < nh) d2 = attach_face(p, nface, nface + g.lane, wi, hreg & 0x3ff, (hreg >> 10) & 0x3ff);
    unsigned long long zero = g.ballot(g.lane < nh && d2 == 0.f);
    int first = zero ? __ffsll((long long)zero) - 1 : nh;
    bool inrange = g.lane < first && d2 >= lower2 && d2 <= upper2;
    if (g.lane < first && !inrange) p.face[nface + g.lane] = face_mark(p.face[nface + g.lane], 0x40000000u);
    nvalid += __popcll(g.ballot(inrange));
    nface += first;
    g.fence();
    if (first < nh) { index = -1; break; }
    if (nvalid == 0) break;
  }
  EpaOut out{kFloatMax, 0, mk(0.f, 0.f, 0.f), mk(0.f, 0.f, 0.f), -1, horizon_overflow, redo};
  if (redo) return out;
  if (g.lane == 0) { p.sc[P_NFACE] = nface; p.sc[P_NVERT] = nvert; }
  if (index >= 0) {
    int packed = p.face[index], ia = packed & 0x3ff, ib = (packed >> 10) & 0x3ff, ic = (packed >> 20) & 0x3ff;
    V wgt = triangle_affine(p.vertex(ia), p.vertex(ib), p.vertex(ic), ld(p.proj + 3 * index));
    out.x1 = wgt[0] * ld(p.vert + 6 * ia) + wgt[1] * ld(p.vert + 6 * ib) + wgt[2] * ld(p.vert + 6 * ic);
    out.x2 = wgt[0] * ld(p.vert + 6 * ia + 3) + wgt[1] * ld(p.vert + 6 * ib + 3) + wgt[2] * ld(p.vert + 6 * ic + 3);
    out.distance = -r_sqrt(p.norm2[index]);
    out.ncontact = 1;
    out.face = index;
  }
  g.fence();
  return out;
}

// ---------------------------------------------------------------- box-box manifold (one lane)
// one[i] - two[i] is the contact normal scaled by |distance[i]|; `dir` is that direction for the
// clipped manifolds (zero for the single EPA point), kept so that the frame does not lose FP32
// precision subtracting two points 1e-4 m apart at positions of order 1 m.
// Small arrays indexed at run time (the clip buffers, the two faces) live in an LDS block of
// kManifoldWords words; the others are only indexed at compile time (unrolled loops with guards,
// pick3 selections), so they stay in registers.
struct Manifold { int count; V one[4], two[4]; real distance[4]; V dir; };
struct Feature { int dim, index[3]; V point[3]; };
struct Normals { int count, index[3]; V normal[3]; };
constexpr int kManifoldWords = 88;
enum : int { MW_FACE1 = 0, MW_FACE2 = 12, MW_NORMAL = 24, MW_PLANE = 36, MW_BUF = 40 };

// a[i] for i < 3 known only at run time
__device__ __forceinline__ V pick3(const V* a, int i) { V r = a[0]; if (i == 1) r = a[1]; if (i == 2) r = a[2]; return r; }
__device__ __forceinline__ int pick3(const int* a, int i) { int r = a[0]; if (i == 1) r = a[1]; if (i == 2) r = a[2]; return r; }

__device__ inline Feature box_feature(const Poly& p, int face, int side) {
  int ids[3] = {face & 1023, (face >> 10) & 1023, (face >> 20) & 1023};
  Feature f;
#pragma unroll
  for (int i = 0; i < 3; ++i) { f.index[i] = p.vidx[2 * ids[i] + side]; f.point[i] = ld(p.vert + 6 * ids[i] + 3 * side); }
  if (f.index[0] != f.index[1]) f.dim = (f.index[2] == f.index[0] || f.index[2] == f.index[1]) ? 2 : 3;
  else { f.index[1] = f.index[2]; f.point[1] = f.point[2]; f.dim = f.index[0] != f.index[2] ? 2 : 1; }
  return f;
}

__device__ __forceinline__ V face_normal(int i) { V n = mk(0.f, 0.f, 0.f); n[i / 2] = (i % 2) == 0 ? 1.f : -1.f; return n; }

__device__ inline Normals normals_near(const CGeom& g, V d) {
  Normals n;
  n.count = 0;
  n.index[0] = n.index[1] = n.index[2] = 0;
  V local = unit(rotT(g.rot, d));
  int hit = -1;
#pragma unroll
  for (int i = 0; i < 6; ++i)
    if (hit < 0 && dot(local, face_normal(i)) > kAlign) hit = i;
  if (hit >= 0) {
    V fn = mk(0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < 6; ++i)
      if (i == hit) fn = face_normal(i);
    n.count = 1; n.normal[0] = rot(g.rot, fn); n.index[0] = hit;
  }
  return n;
}

__device__ inline Normals box_normals(const CGeom& g, const Feature& f, V d) {
  Normals n;
  n.count = 0;
  n.index[0] = n.index[1] = n.index[2] = 0;
  if (f.dim == 3) {
    V common = mk(0.f, 0.f, 0.f);
    int count = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      int bit = 1 << k;
      real value = real((f.index[0] & bit) && (f.index[1] & bit) && (f.index[2] & bit)) -
                    real(!(f.index[0] & bit) && !(f.index[1] & bit) && !(f.index[2] & bit));
      common[k] = value;
      if (value != 0.f) {
#pragma unroll
        for (int s = 0; s < 3; ++s)
          if (s == count) n.index[s] = 2 * k;
        ++count;
      }
    }
    if (common[0] + common[1] + common[2] == -1.f) ++n.index[0];
    if (count == 1) { n.count = 1; n.normal[0] = rot(g.rot, common); return n; }
    return normals_near(g, d);
  }
  if (f.dim == 2) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      int bit = 1 << k;
      real value = real((f.index[0] & bit) && (f.index[1] & bit)) - real(!(f.index[0] & bit) && !(f.index[1] & bit));
      if (value != 0.f) {
        V local = mk(0.f, 0.f, 0.f);
        local[k] = value;
        V nv = rot(g.rot, local);
#pragma unroll
        for (int s = 0; s < 3; ++s)
          if (s == n.count) { n.normal[s] = nv; n.index[s] = 2 * k + (value > 0.f ? 0 : 1); }
        ++n.count;
      }
    }
    if (n.count == 1 || n.count == 2) return n;
    return normals_near(g, d);
  }
  if (f.dim == 1) {
    n.count = 3;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      int i = 2 * k + ((f.index[0] & (1 << k)) ? 0 : 1);
      n.index[k] = i;
      n.normal[k] = rot(g.rot, face_normal(i));
    }
  }
  return n;
}

__device__ inline Normals edge_normals(const CGeom& g, const Feature& f, V* end) {
  Normals n;
  n.count = 0;
  n.index[0] = n.index[1] = n.index[2] = 0;
  if (f.dim == 2) { end[0] = f.point[1]; n.normal[0] = unit(f.point[1] - f.point[0]); n.count = 1; }
  if (f.dim == 1) {
    V local;
#pragma unroll
    for (int k = 0; k < 3; ++k) local[k] = (f.index[0] & (1 << k)) ? g.size[k] : -g.size[k];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      V pt = local;
      pt[k] = -pt[k];
      end[k] = rot(g.rot, pt) + g.pos;
      n.normal[k] = unit(end[k] - f.point[0]);
    }
    n.count = 3;
  }
  return n;
}

// the four corners of box face `face` (0..5), world frame, into out (12 words)
__device__ inline int box_face(const CGeom& g, int face, sreal* out) {
  const int corners[6][4] = {{7, 3, 1, 5}, {2, 6, 4, 0}, {2, 3, 7, 6}, {4, 5, 1, 0}, {6, 7, 5, 4}, {3, 2, 0, 1}};
  int cs[4] = {0, 0, 0, 0};
#pragma unroll
  for (int fc = 0; fc < 6; ++fc)
    if (fc == face) {
#pragma unroll
      for (int i = 0; i < 4; ++i) cs[i] = corners[fc][i];
    }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    V pt;
#pragma unroll
    for (int k = 0; k < 3; ++k) pt[k] = (cs[i] & (1 << k)) ? g.size[k] : -g.size[k];
    st(out + 3 * i, rot(g.rot, pt) + g.pos);
  }
  return 4;
}

__device__ __forceinline__ real quad_area(V a, V b, V c, V d) { V n = crs(a - c, b - d); return 0.5f * r_sqrt(dot(n, n)); }

// the polygon's points are 3 words apart in LDS
__device__ inline void polygon_quad(const sreal* p, int count, int* res) {
  auto P = [&](int i) { return ld(p + 3 * i); };
  int b = 1, c = 2, d = 3;
  res[0] = 0; res[1] = b; res[2] = c; res[3] = d;
  real area = quad_area(P(0), P(b), P(c), P(d));
  for (int a = 0; a < count; ++a) {
    while (true) {
      real next = quad_area(P(a), P(b), P(c), P((d + 1) % count));
      if (next <= area) break;
      area = next; d = (d + 1) % count;
      res[0] = a; res[1] = b; res[2] = c; res[3] = d;
      while (true) {
        next = quad_area(P(a), P(b), P((c + 1) % count), P(d));
        if (next <= area) break;
        area = next; c = (c + 1) % count;
        res[0] = a; res[1] = b; res[2] = c; res[3] = d;
      }
      while (true) {
        next = quad_area(P(a), P((b + 1) % count), P(c), P(d));
        if (next <= area) break;
        area = next; b = (b + 1) % count;
        res[0] = a; res[1] = b; res[2] = c; res[3] = d;
      }
    }
    if (b == a) {
      b = (b + 1) % count;
      if (c == b) { c = (c + 1) % count; if (d == c) d = (d + 1) % count; }
    }
  }
}

// clip polygon face2 (n2 points) against the side planes of face1 (n1 points); both in LDS
__device__ inline Manifold polygon_clip(const sreal* face1, int n1, const sreal* face2, int n2, V normal, V direction,
                                        sreal* ws) {
  Manifold res;
  res.count = 0;
  res.dir = -direction;
  if (n1 < 3) return res;
  sreal* normals = ws + MW_NORMAL;
  sreal* plane = ws + MW_PLANE;
  sreal* buf[2] = {ws + MW_BUF, ws + MW_BUF + 24};
  auto F1 = [&](int i) { return ld(face1 + 3 * i); };
  for (int i = 0; i < n1; ++i) {
    V fi = F1(i), nrm = crs(F1((i + 1) % n1) - fi, (fi + normal) - fi);
    st(normals + 3 * i, nrm);
    plane[i] = dot(nrm, fi);
  }
  int cur = 0;
  int count = n2;
  for (int i = 0; i < n2; ++i) st(buf[0] + 3 * i, ld(face2 + 3 * i));
  for (int e = 0; e < n1; ++e) {
    int nc = 0;
    const sreal* poly = buf[cur];
    sreal* clipped = buf[cur ^ 1];
    V fe = F1(e), ne = ld(normals + 3 * e);
    real pe = plane[e];
    for (int i = 0; i < count; ++i) {
      V p = ld(poly + 3 * i), q = ld(poly + 3 * ((i + 1) % count));
      bool in1 = dot(p - fe, ne) > -1e-10f, in2 = dot(q - fe, ne) > -1e-10f;
      if (!in1 && !in2) continue;
      if (in1 && in2) { if (nc < 8) st(clipped + 3 * nc++, q); continue; }
      real den = dot(ne, q - p);
      real t = r_abs(den) < 1e-10f ? kFloatMax : (pe - dot(ne, p)) / den;
      if (t > -3e-7f && t < 1.f + 3e-7f && nc < 8) { t = r_min(1.f, r_max(0.f, t)); st(clipped + 3 * nc++, p + t * (q - p)); }
      if (in2 && nc < 8) st(clipped + 3 * nc++, q);
    }
    cur ^= 1;
    count = nc;
  }
  sreal* poly = buf[cur];
  V f0 = F1(0);
  int kept = 0;
  for (int i = 0; i < count; ++i) {
    V v = ld(poly + 3 * i);
    if (dot(v - f0, normal) <= 0.f) st(poly + 3 * kept++, v);
  }
  count = kept;
  if (count < 1) return res;
  int ids[4] = {0, 1, 2, 3};
  if (n2 == 2 && count > 2) {
    real mx = 0.f;
    ids[0] = 0; ids[1] = 1;
    for (int i = 0; i < count; ++i)
      for (int j = i + 1; j < count; ++j) {
        V d = ld(poly + 3 * j) - ld(poly + 3 * i);
        real l = dot(d, d);
        if (l > mx) { mx = l; ids[0] = i; ids[1] = j; }
      }
    res.count = 2;
  } else if (count > 4) {
    polygon_quad(poly, count, ids);
    res.count = 4;
  } else {
    res.count = count;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i >= res.count) continue;
    V v = ld(poly + 3 * ids[i]);
    real d = dot(v - f0, normal);
    res.one[i] = v - direction * r_abs(d);
    res.two[i] = v;
    res.distance[i] = d;
  }
  return res;
}

// ws: kManifoldWords words of LDS
__device__ inline Manifold box_multicontact(const Poly& p, int face, V x1, V x2, const CGeom& a, const CGeom& b,
                                            sreal* ws) {
  Manifold fallback;
  fallback.count = 1; fallback.one[0] = x1; fallback.two[0] = x2; fallback.dir = mk(0.f, 0.f, 0.f);
  Feature one = box_feature(p, p.face[face], 0), two = box_feature(p, p.face[face], 1);
  V dir = x2 - x1, end[3];
  Normals n1 = box_normals(a, one, -dir), n2 = box_normals(b, two, dir);
  int i = 0, j = 0, edge1 = 0, edge2 = 0;
  bool aligned = false;
  // the first (k, l) in order whose normals oppose
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int l = 0; l < 3; ++l)
      if (!aligned && k < n1.count && l < n2.count && dot(n1.normal[k], n2.normal[l]) < -kAlign) {
        i = k; j = l; aligned = true;
      }
  if (!aligned) {
    if (one.dim < 3 && n2.count && (one.dim <= two.dim || !n1.count)) {
      n1 = edge_normals(a, one, end);
#pragma unroll
      for (int k = 0; k < 3; ++k)
#pragma unroll
        for (int l = 0; l < 3; ++l)
          if (!aligned && k < n2.count && l < n1.count && !(dot(n2.normal[k], dir) <= kConvexMin) &&
              r_abs(dot(n1.normal[l], n2.normal[k])) < kPerp) {
            i = l; j = k; aligned = true;
          }
      if (!aligned) return fallback;
      edge1 = 1;
    } else if (two.dim < 3) {
      n2 = edge_normals(b, two, end);
#pragma unroll
      for (int k = 0; k < 3; ++k)
#pragma unroll
        for (int l = 0; l < 3; ++l)
          if (!aligned && k < n1.count && l < n2.count && !(dot(n1.normal[k], -dir) <= kConvexMin) &&
              r_abs(dot(n2.normal[l], n1.normal[k])) < kPerp) {
            i = l; j = k; aligned = true;
          }
      if (!aligned) return fallback;
      edge2 = 1;
    } else {
      return fallback;
    }
  }
  sreal* face1 = ws + MW_FACE1;
  sreal* face2 = ws + MW_FACE2;
  int c1, c2;
  if (edge1) { st(face1, one.point[0]); st(face1 + 3, pick3(end, i)); c1 = 2; }
  else c1 = box_face(a, pick3(n1.index, edge2 ? j : i), face1);
  if (edge2) { st(face2, two.point[0]); st(face2 + 3, pick3(end, i)); c2 = 2; }
  else c2 = box_face(b, pick3(n2.index, j), face2);
  if (edge1) {
    V nj = pick3(n2.normal, j);
    Manifold r = polygon_clip(face2, c2, face1, c1, nj, -nj, ws);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (k >= r.count) continue;
      V t = r.one[k]; r.one[k] = r.two[k]; r.two[k] = t;
    }
    r.dir = -r.dir;
    return r;
  }
  if (edge2) { V nj = pick3(n1.normal, j); return polygon_clip(face1, c1, face2, c2, nj, -nj, ws); }
  return polygon_clip(face1, c1, face2, c2, pick3(n1.normal, i), pick3(n2.normal, j), ws);
}

__device__ __forceinline__ bool multicontact_supported(const CGeom& a, const CGeom& b) {
  if (a.margin != 0.f || b.margin != 0.f) return false;
  bool f1 = a.type == GT_BOX || a.type == GT_MESH, f2 = b.type == GT_BOX || b.type == GT_MESH;
  return (f1 && f2) || (a.type == GT_CAPSULE && f2) || (f1 && b.type == GT_CAPSULE);
}

// EPA's single contact: the witness points and, as `dir`, the projection of the origin onto the
// result face (x1 - x2 is that projection in exact arithmetic).  The face normal comes from edges of
// the polytope, the witness difference from sums of support points that can lie a geom's extent
// from the origin: with a penetration of 1e-4 m and support points 1 m out, their FP32 rounding
// turns the normalized difference by up to 1e-3, the face normal by 1e-7.
__device__ inline Manifold single_point(const EpaOut& e, V face_proj) {
  Manifold mf;
  mf.count = e.ncontact;
  mf.one[0] = e.x1;
  mf.two[0] = e.x2;
  mf.distance[0] = e.distance;
  mf.dir = face_proj;
  return mf;
}

// Contacts of a finished convex pair (one lane): the manifold for box-box, else one point.
// x1, x2 are in the pair's translated frame (origin: pair_origin).
__device__ inline void emit(RawOut& __restrict__ o, const Manifold& __restrict__ mf, real distance, real margin, real thr, V origin) {
  // the reference normalizes one[0] - two[0] (mjwarp_convex_collision.cuh:74); for a clipped
  // manifold with nonzero depth that difference is exactly |distance[0]| dir, and for EPA's single
  // point it is the result face's projection of the origin (single_point)
  V diff = mf.one[0] - mf.two[0];
  if (mf.count > 0 && mf.distance[0] != 0.f && dot(mf.dir, mf.dir) > 0.f) diff = mf.dir;
  V n = unit(distance <= margin ? diff : -diff);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i >= mf.count) continue;
    real d = mf.count > 1 ? mf.distance[i] : distance;
    if (!(d < thr)) continue;
    V pos = 0.5f * (mf.one[i] + mf.two[i]) + origin;
    raw_push(o, pos.v, n.v, d);
  }
}


// ---------------------------------------------------------------- MPR (MuJoCo 2.3.7)
// The MPR steps below restate libccd's ccdMPRPenetration, which carries this notice:
//
//   libccd
//   Copyright (c)2010-2012 Daniel Fiser <danfis@danfis.cz>,
//   Intelligent and Mobile Robotics Group, Department of Cybernetics,
//   Faculty of Electrical Engineering, Czech Technical University in Prague.
//   All rights reserved.
//
//   Redistribution and use in source and binary forms, with or without
//   modification, are permitted provided that the following conditions are met:
//    - Redistributions of source code must retain the above copyright notice,
//      this list of conditions and the following disclaimer.
//    - Redistributions in binary form must reproduce the above copyright
//      notice, this list of conditions and the following disclaimer in the
//      documentation and/or other materials provided with the distribution.
//    - Neither the name of the University nor the names of its contributors
//      may be used to endorse or promote products derived from this software
//      without specific prior written permission.
//
//   THIS SOFTWARE IS PROVIDED BY THE COPYRIGHT HOLDERS AND CONTRIBUTORS "AS IS"
//   AND ANY EXPRESS OR IMPLIED WARRANTIES, INCLUDING, BUT NOT LIMITED TO, THE
//   IMPLIED WARRANTIES OF MERCHANTABILITY AND FITNESS FOR A PARTICULAR PURPOSE
//   ARE DISCLAIMED. IN NO EVENT SHALL THE COPYRIGHT HOLDER OR CONTRIBUTORS BE
//   LIABLE FOR ANY DIRECT, INDIRECT, INCIDENTAL, SPECIAL, EXEMPLARY, OR
//   CONSEQUENTIAL DAMAGES (INCLUDING, BUT NOT LIMITED TO, PROCUREMENT OF
//   SUBSTITUTE GOODS OR SERVICES; LOSS OF USE, DATA, OR PROFITS; OR BUSINESS
//   INTERRUPTION) HOWEVER CAUSED AND ON ANY THEORY OF LIABILITY, WHETHER IN
//   CONTRACT, STRICT LIABILITY, OR TORT (INCLUDING NEGLIGENCE OR OTHERWISE)
//   ARISING IN ANY WAY OUT OF THE USE OF THIS SOFTWARE, EVEN IF ADVISED OF THE
//   POSSIBILITY OF SUCH DAMAGE.
//
// One convex pair by Minkowski Portal Refinement on one lane, MuJoCo 2.3.7's mjc_Convex with
// multiccd off: libccd's ccdMPRPenetration in its float build (zero and equality tests against
// FLT_EPSILON), MuJoCo's support points (a box coordinate sign(d) size with sign(0) = 0, a hull's
// first vertex of largest projection), the contact at the mean of the portal's support points.
// Restated from the algorithm as vendored by the reference in
// gpu/host/runtime/collision/native_originals/ (ccd_mpr.c.txt, ccd_vec3.c.txt:73-216,
// engine_collision_convex.c.txt:42-240).  Portal discovery and refinement are bounded by the
// iteration count (the originals loop until they decide), so every lane's loop ends.
namespace mpr {
constexpr real kEps = 1.1920928955078125e-7f;
__device__ __forceinline__ bool zero(real x) { return r_abs(x) < kEps; }
__device__ __forceinline__ bool eq(real a, real b) {
  real ab = r_abs(a - b);
  return ab < kEps || ab < kEps * r_max(r_abs(a), r_abs(b));
}
__device__ __forceinline__ bool at_origin(V a) { return eq(a[0], 0.f) && eq(a[1], 0.f) && eq(a[2], 0.f); }
__device__ __forceinline__ V norm(V a) { return a * (1.f / r_sqrt(dot(a, a))); }
struct Sup { V v, v1, v2; };

__device__ inline V point(const CGeom& g, V d) {
  if (g.type == GT_SPHERE) return g.pos + (g.size[0] + 0.5f * g.margin) * d;
  V local = rotT(g.rot, d), res = mk(0.f, 0.f, 0.f);
  if (g.type == GT_BOX) {
    for (int k = 0; k < 3; ++k) res[k] = sgn(local[k]) * g.size[k];
  } else if (g.type == GT_CAPSULE) {
    res = local * g.size[0];
    res[2] += sgn(local[2]) * g.size[1];
  } else if (g.type == GT_MESH) {
    real best = -1e10f;
    for (int i0 = 0; i0 < g.nvert; i0 += 4) {   // ascending, four vertices' loads issued together
      v4f q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) q[u] = *(const sfloat4*)(g.vert + 4 * (i0 + u < g.nvert ? i0 + u : i0));
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (i0 + u >= g.nvert) continue;
        V v = mk(q[u].x, q[u].y, q[u].z);
        real h = dot(v, local);
        if (h > best) { best = h; res = v; }
      }
    }
  }
  res = res + local * (0.5f * g.margin);
  return rot(g.rot, res) + g.pos;
}
__device__ __forceinline__ Sup sup(const CGeom& a, const CGeom& b, V d) {
  Sup s;
  s.v1 = point(a, d);
  s.v2 = point(b, -d);
  s.v = s.v1 - s.v2;
  return s;
}
__device__ __forceinline__ V portal_dir(const Sup* p) { return norm(crs(p[2].v - p[1].v, p[3].v - p[1].v)); }
__device__ __forceinline__ bool reach_tolerance(const Sup* p, const Sup& v4, V dir, real tol) {
  real d4 = dot(v4.v, dir);
  real m = r_min(d4 - dot(p[1].v, dir), r_min(d4 - dot(p[2].v, dir), d4 - dot(p[3].v, dir)));
  return eq(m, tol) || m < tol;
}
__device__ __forceinline__ void expand(Sup* p, const Sup& v4) {
  V c = crs(v4.v, p[0].v);
  if (dot(p[1].v, c) > 0.f) {
    if (dot(p[2].v, c) > 0.f) p[1] = v4; else p[3] = v4;
  } else {
    if (dot(p[3].v, c) > 0.f) p[2] = v4; else p[1] = v4;
  }
}
__device__ inline real seg_dist2(V x0, V b, V& w) {
  V d = b - x0;
  real t = -dot(x0, d) / dot(d, d);
  if (t < 0.f || zero(t)) w = x0;
  else if (t > 1.f || eq(t, 1.f)) w = b;
  else w = x0 + t * d;
  return dot(w, w);
}
__device__ inline real tri_dist2(V x0, V b, V c, V& w) {
  V d1 = b - x0, d2 = c - x0;
  real v = dot(d1, d1), ww = dot(d2, d2), p = dot(x0, d1), q = dot(x0, d2), r = dot(d1, d2);
  real d = ww * v - r * r, s, t;
  if (zero(d)) { s = t = -1.f; }
  else { s = (q * r - ww * p) / d; t = (-s * r - q) / ww; }
  if ((zero(s) || s > 0.f) && (eq(s, 1.f) || s < 1.f) && (zero(t) || t > 0.f) && (eq(t, 1.f) || t < 1.f) &&
      (eq(t + s, 1.f) || t + s < 1.f)) {
    w = x0 + s * d1 + t * d2;
    return dot(w, w);
  }
  V w2;
  real dist = seg_dist2(x0, b, w), e = seg_dist2(x0, c, w2);
  if (e < dist) { dist = e; w = w2; }
  e = seg_dist2(b, c, w2);
  if (e < dist) { dist = e; w = w2; }
  return dist;
}
__device__ inline V portal_pos(const Sup* p) {
  V dir = portal_dir(p);
  real b0 = dot(crs(p[1].v, p[2].v), p[3].v), b1 = dot(crs(p[3].v, p[2].v), p[0].v);
  real b2 = dot(crs(p[0].v, p[1].v), p[3].v), b3 = dot(crs(p[2].v, p[1].v), p[0].v);
  real sum = b0 + b1 + b2 + b3;
  if (zero(sum) || sum < 0.f) {
    b0 = 0.f;
    b1 = dot(crs(p[2].v, p[3].v), dir);
    b2 = dot(crs(p[3].v, p[1].v), dir);
    b3 = dot(crs(p[1].v, p[2].v), dir);
    sum = b1 + b2 + b3;
  }
  const real inv = 1.f / sum;
  V p1 = b0 * p[0].v1 + b1 * p[1].v1 + b2 * p[2].v1 + b3 * p[3].v1;
  V p2 = b0 * p[0].v2 + b1 * p[1].v2 + b2 * p[2].v2 + b3 * p[3].v2;
  return 0.5f * (p1 * inv + p2 * inv);
}
// true with the depth, normal and point (the geoms' frame) when the geoms penetrate; a touching
// contact (no normal) counts as none, as in MuJoCo's caller
__device__ inline bool penetration(const CGeom& a, const CGeom& b, real tol, int maxit, real& depth, V& dir, V& pos) {
  Sup p[4];
  p[0].v1 = a.pos; p[0].v2 = b.pos; p[0].v = a.pos - b.pos;
  if (at_origin(p[0].v)) p[0].v[0] += kEps * 10.f;
  V d = norm(-p[0].v);
  p[1] = sup(a, b, d);
  real dt = dot(p[1].v, d);
  if (zero(dt) || dt < 0.f) return false;
  d = crs(p[0].v, p[1].v);
  if (zero(dot(d, d))) {
    if (at_origin(p[1].v)) return false;      // touching at v1: no normal
    pos = 0.5f * (p[1].v1 + p[1].v2);         // origin on segment v0-v1
    depth = r_sqrt(dot(p[1].v, p[1].v));
    dir = norm(p[1].v);
    return !at_origin(dir);
  }
  d = norm(d);
  p[2] = sup(a, b, d);
  dt = dot(p[2].v, d);
  if (zero(dt) || dt < 0.f) return false;
  d = norm(crs(p[1].v - p[0].v, p[2].v - p[0].v));
  if (dot(d, p[0].v) > 0.f) { Sup t = p[1]; p[1] = p[2]; p[2] = t; d = -d; }
  bool built = false;
  for (int it = 0; it < maxit && !built; ++it) {
    p[3] = sup(a, b, d);
    dt = dot(p[3].v, d);
    if (zero(dt) || dt < 0.f) return false;
    bool cont = false;
    dt = dot(crs(p[1].v, p[3].v), p[0].v);
    if (dt < 0.f && !zero(dt)) { p[2] = p[3]; cont = true; }
    if (!cont) {
      dt = dot(crs(p[3].v, p[2].v), p[0].v);
      if (dt < 0.f && !zero(dt)) { p[1] = p[3]; cont = true; }
    }
    if (cont) d = norm(crs(p[1].v - p[0].v, p[2].v - p[0].v));
    else built = true;
  }
  if (!built) return false;
  bool enclosed = false;
  for (int it = 0; it < maxit && !enclosed; ++it) {   // refine until the portal encloses the origin
    d = portal_dir(p);
    real e = dot(d, p[1].v);
    if (zero(e) || e > 0.f) { enclosed = true; break; }
    Sup v4 = sup(a, b, d);
    real c4 = dot(v4.v, d);
    if (!(zero(c4) || c4 > 0.f) || reach_tolerance(p, v4, d, tol)) return false;
    expand(p, v4);
  }
  if (!enclosed) return false;
  for (int it = 0;; ++it) {   // expand towards the boundary; ends by tolerance or by count
    d = portal_dir(p);
    Sup v4 = sup(a, b, d);
    if (reach_tolerance(p, v4, d, tol) || it > maxit) {
      V w;
      depth = r_sqrt(tri_dist2(p[1].v, p[2].v, p[3].v, w));
      if (zero(depth)) return false;           // no normal: none
      dir = norm(w);
      pos = portal_pos(p);
      return true;
    }
    expand(p, v4);
  }
}
}  // namespace mpr
}  // namespace cvx
}  // namespace mx
