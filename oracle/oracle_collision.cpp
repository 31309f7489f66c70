// Collision detection of the CPU FP64 oracle -- TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// Broadphase over the model's static pair table (bounding spheres, plane half-space), then one
// narrowphase routine per geom-type pair, restating:
//   plane-*            gpu/cuda/collision/mjwarp_plane.cu:120-141 (sphere, capsule, box corners, mesh)
//   box-box            SAT over 15 axes + incident-face clipping (the role of mjwarp_box.cu:115-176
//                      and mjwarp_box_manifold.cuh:105-133; fixtures tests/fixtures/boxbox_*)
//   capsule-box        segment vs box (mjwarp_box.cu:33-102)
//   capsule-capsule    segment-segment closest points (absent in the reference, MuJoCo semantics)
//   sphere-*           closed forms (mjwarp_box.cu:14-32)
//   mesh-*             GJK distance / EPA penetration + face clipping (mjwarp_convex_*.cuh)
// Contact convention (MuJoCo): the normal points from geom1 to geom2, pos is the midpoint between
// the surfaces, dist < 0 is penetration.  Material mixing restates contact_material
// (gpu/cuda/collision/mjwarp_contact.cuh:56-101); the frame restates MJWarp's make_frame.
#include "oracle_internal.h"

namespace orc {
namespace {

enum { PLANE = 0, SPHERE = 2, CAPSULE = 3, BOX = 6, MESH = 7 };

struct Geom {
  int id, type;
  T pos[3], mat[9], size[3];
  const T* vert = nullptr;
  int nvert = 0;
};

struct Raw {   // one contact before material assignment
  T pos[3], normal[3], dist;
};

void axis(const T* mat, int k, T* out) { out[0] = mat[k]; out[1] = mat[3 + k]; out[2] = mat[6 + k]; }

void normalize3(T* v) {
  T n = norm3(v);
  if (n > kMinVal) { v[0] /= n; v[1] /= n; v[2] /= n; }
}

// MJWarp make_frame: tangent from y (or z when the normal is close to y), then the cross product.
void make_frame(const T* n, T* frame) {
  T a[3] = {n[0], n[1], n[2]};
  normalize3(a);
  T b[3];
  if (-0.5 < a[1] && a[1] < 0.5) { b[0] = 0; b[1] = 1; b[2] = 0; }
  else { b[0] = 0; b[1] = 0; b[2] = 1; }
  T d = dot3(a, b);
  for (int k = 0; k < 3; ++k) b[k] -= a[k] * d;
  normalize3(b);
  T c[3];
  cross(a, b, c);
  for (int k = 0; k < 3; ++k) { frame[k] = a[k]; frame[3 + k] = b[k]; frame[6 + k] = c[k]; }
}

void push(std::vector<Raw>& out, const T* pos, const T* normal, T dist) {
  Raw r;
  for (int k = 0; k < 3; ++k) { r.pos[k] = pos[k]; r.normal[k] = normal[k]; }
  r.dist = dist;
  out.push_back(r);
}

// ------------------------------------------------------------------ plane
void plane_point(const Geom& p, const T* c, T r, T margin, std::vector<Raw>& out) {
  T n[3];
  axis(p.mat, 2, n);
  T d[3] = {c[0] - p.pos[0], c[1] - p.pos[1], c[2] - p.pos[2]};
  T dist = dot3(n, d) - r;
  if (dist >= margin) return;
  T pos[3];
  for (int k = 0; k < 3; ++k) pos[k] = c[k] - n[k] * (r + 0.5 * dist);
  push(out, pos, n, dist);
}

// up to 4 deepest of a vertex set below the plane
void plane_vertices(const Geom& p, const std::vector<std::array<T, 3>>& verts, T margin, std::vector<Raw>& out) {
  T n[3];
  axis(p.mat, 2, n);
  std::vector<std::pair<T, int>> below;
  for (int i = 0; i < (int)verts.size(); ++i) {
    T d[3] = {verts[i][0] - p.pos[0], verts[i][1] - p.pos[1], verts[i][2] - p.pos[2]};
    T dist = dot3(n, d);
    if (dist < margin) below.push_back({dist, i});
  }
  std::stable_sort(below.begin(), below.end(), [](const std::pair<T, int>& a, const std::pair<T, int>& b) {
    return a.first < b.first;
  });
  for (int k = 0; k < (int)below.size() && k < 4; ++k) {
    const auto& v = verts[below[k].second];
    T dist = below[k].first, pos[3];
    for (int j = 0; j < 3; ++j) pos[j] = v[j] - n[j] * 0.5 * dist;
    push(out, pos, n, dist);
  }
}

std::vector<std::array<T, 3>> box_corners(const Geom& g) {
  std::vector<std::array<T, 3>> v(8);
  for (int i = 0; i < 8; ++i) {
    T l[3] = {(i & 1) ? g.size[0] : -g.size[0], (i & 2) ? g.size[1] : -g.size[1], (i & 4) ? g.size[2] : -g.size[2]};
    T w[3];
    mulmv3(g.mat, l, w);
    for (int k = 0; k < 3; ++k) v[i][k] = g.pos[k] + w[k];
  }
  return v;
}

std::vector<std::array<T, 3>> mesh_world(const Geom& g) {
  std::vector<std::array<T, 3>> v(g.nvert);
  for (int i = 0; i < g.nvert; ++i) {
    T w[3];
    mulmv3(g.mat, g.vert + 3 * i, w);
    for (int k = 0; k < 3; ++k) v[i][k] = g.pos[k] + w[k];
  }
  return v;
}

void segment(const Geom& g, T* a, T* b) {
  T ax[3];
  axis(g.mat, 2, ax);
  for (int k = 0; k < 3; ++k) { a[k] = g.pos[k] - g.size[1] * ax[k]; b[k] = g.pos[k] + g.size[1] * ax[k]; }
}

// ------------------------------------------------------------------ spheres and segments
void sphere_sphere(const T* c1, T r1, const T* c2, T r2, T margin, std::vector<Raw>& out, const T* fallback) {
  T d[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
  T len = norm3(d);
  T dist = len - r1 - r2;
  if (dist >= margin) return;
  T n[3];
  if (len > kMinVal) { for (int k = 0; k < 3; ++k) n[k] = d[k] / len; }
  else { for (int k = 0; k < 3; ++k) n[k] = fallback[k]; }
  T pos[3];
  for (int k = 0; k < 3; ++k) pos[k] = c1[k] + n[k] * (r1 + 0.5 * dist);
  push(out, pos, n, dist);
}

// closest points between segments [p1,q1] and [p2,q2] (clamped parameters s, t)
void closest_segments(const T* p1, const T* q1, const T* p2, const T* q2, T& s, T& t) {
  T d1[3], d2[3], r[3];
  for (int k = 0; k < 3; ++k) { d1[k] = q1[k] - p1[k]; d2[k] = q2[k] - p2[k]; r[k] = p1[k] - p2[k]; }
  T a = dot3(d1, d1), e = dot3(d2, d2), f = dot3(d2, r);
  if (a <= kMinVal && e <= kMinVal) { s = t = 0; return; }
  if (a <= kMinVal) { s = 0; t = std::min(std::max(f / e, T(0)), T(1)); return; }
  T c = dot3(d1, r);
  if (e <= kMinVal) { t = 0; s = std::min(std::max(-c / a, T(0)), T(1)); return; }
  T b = dot3(d1, d2), denom = a * e - b * b;
  s = denom > kMinVal * a * e ? std::min(std::max((b * f - c * e) / denom, T(0)), T(1)) : 0;
  t = (b * s + f) / e;
  if (t < 0) { t = 0; s = std::min(std::max(-c / a, T(0)), T(1)); }
  else if (t > 1) { t = 1; s = std::min(std::max((b - c) / a, T(0)), T(1)); }
}

void capsule_capsule(const Geom& g1, const Geom& g2, T margin, std::vector<Raw>& out) {
  T a1[3], b1[3], a2[3], b2[3];
  segment(g1, a1, b1);
  segment(g2, a2, b2);
  T r1 = g1.size[0], r2 = g2.size[0];
  T d1[3], d2[3], cr[3];
  for (int k = 0; k < 3; ++k) { d1[k] = b1[k] - a1[k]; d2[k] = b2[k] - a2[k]; }
  cross(d1, d2, cr);
  T l1 = norm3(d1), l2 = norm3(d2);
  T fallback[3];
  cross(d1, d2, fallback);
  if (norm3(fallback) < kMinVal) { fallback[0] = 0; fallback[1] = 0; fallback[2] = 1; }
  normalize3(fallback);
  if (l1 > kMinVal && l2 > kMinVal && norm3(cr) < 1e-3 * l1 * l2) {
    // (nearly) parallel: contacts at both ends of the overlap of segment 2 projected on segment 1
    T u[3] = {d1[0] / l1, d1[1] / l1, d1[2] / l1};
    T ta[3] = {a2[0] - a1[0], a2[1] - a1[1], a2[2] - a1[2]}, tb[3] = {b2[0] - a1[0], b2[1] - a1[1], b2[2] - a1[2]};
    T s0 = dot3(ta, u), s1 = dot3(tb, u);
    T lo = std::max(std::min(s0, s1), T(0)), hi = std::min(std::max(s0, s1), l1);
    if (hi - lo > 1e-6 * l1) {
      for (T sp : {lo, hi}) {
        T p1[3], p2[3];
        for (int k = 0; k < 3; ++k) p1[k] = a1[k] + u[k] * sp;
        T t = (sp - s0) / (s1 - s0);
        t = std::min(std::max(t, T(0)), T(1));
        for (int k = 0; k < 3; ++k) p2[k] = a2[k] + d2[k] * t;
        sphere_sphere(p1, r1, p2, r2, margin, out, fallback);
      }
      return;
    }
  }
  T s, t;
  closest_segments(a1, b1, a2, b2, s, t);
  T p1[3], p2[3];
  for (int k = 0; k < 3; ++k) { p1[k] = a1[k] + d1[k] * s; p2[k] = a2[k] + d2[k] * t; }
  sphere_sphere(p1, r1, p2, r2, margin, out, fallback);
}

// signed distance from point p to box g; closest point on the surface and the outward normal there
T point_box(const Geom& g, const T* p, T* normal) {
  T d[3] = {p[0] - g.pos[0], p[1] - g.pos[1], p[2] - g.pos[2]}, l[3];
  mulmtv3(g.mat, d, l);
  bool inside = true;
  T c[3];
  for (int k = 0; k < 3; ++k) {
    c[k] = std::min(std::max(l[k], -g.size[k]), g.size[k]);
    inside &= std::fabs(l[k]) <= g.size[k];
  }
  if (!inside) {
    T diff[3] = {l[0] - c[0], l[1] - c[1], l[2] - c[2]};
    T len = norm3(diff);
    T nl[3] = {diff[0] / len, diff[1] / len, diff[2] / len};
    mulmv3(g.mat, nl, normal);
    return len;
  }
  int best = 0;
  T gap = g.size[0] - std::fabs(l[0]);
  for (int k = 1; k < 3; ++k)
    if (g.size[k] - std::fabs(l[k]) < gap) { gap = g.size[k] - std::fabs(l[k]); best = k; }
  T nl[3] = {0, 0, 0};
  nl[best] = l[best] >= 0 ? 1 : -1;
  mulmv3(g.mat, nl, normal);
  return -gap;
}

// sphere (c, r) as geom1 against box geom2: normal from the sphere to the box
void sphere_box(const T* c, T r, const Geom& box, T margin, std::vector<Raw>& out) {
  T nb[3];
  T sd = point_box(box, c, nb);
  T dist = sd - r;
  if (dist >= margin) return;
  T n[3] = {-nb[0], -nb[1], -nb[2]}, pos[3];
  for (int k = 0; k < 3; ++k) pos[k] = c[k] + n[k] * (r + 0.5 * dist);
  push(out, pos, n, dist);
}

void capsule_box(const Geom& cap, const Geom& box, T margin, std::vector<Raw>& out) {
  T a[3], b[3];
  segment(cap, a, b);
  T r = cap.size[0];
  auto at = [&](T t, T* p) { for (int k = 0; k < 3; ++k) p[k] = a[k] + (b[k] - a[k]) * t; };
  auto f = [&](T t) { T p[3], n[3]; at(t, p); return point_box(box, p, n); };
  // endpoints first; the interior minimum of the (convex) distance only when an end is not touching
  std::vector<Raw> ends;
  T pa[3], pb[3];
  at(0, pa);
  at(1, pb);
  sphere_box(pa, r, box, margin, ends);
  sphere_box(pb, r, box, margin, ends);
  if (ends.size() == 2) { out.insert(out.end(), ends.begin(), ends.end()); return; }
  T lo = 0, hi = 1;
  for (int it = 0; it < 60; ++it) {
    T m1 = lo + (hi - lo) / 3, m2 = hi - (hi - lo) / 3;
    if (f(m1) <= f(m2)) hi = m2; else lo = m1;
  }
  T tm = 0.5 * (lo + hi);
  out.insert(out.end(), ends.begin(), ends.end());
  if (tm > 1e-3 && tm < 1 - 1e-3) {
    T pm[3];
    at(tm, pm);
    sphere_box(pm, r, box, margin, out);
  }
}

// ------------------------------------------------------------------ box-box: SAT + clipping
// Reduce a point set to at most 4: deepest, farthest from it, largest triangle, largest quad.
void reduce4(std::vector<Raw>& pts) {
  if (pts.size() <= 4) return;
  std::vector<Raw> keep;
  int n = (int)pts.size();
  std::vector<bool> used(n, false);
  int i0 = 0;
  for (int i = 1; i < n; ++i) if (pts[i].dist < pts[i0].dist) i0 = i;
  used[i0] = true;
  keep.push_back(pts[i0]);
  int i1 = -1;
  T best = -1;
  for (int i = 0; i < n; ++i) {
    if (used[i]) continue;
    T d[3] = {pts[i].pos[0] - pts[i0].pos[0], pts[i].pos[1] - pts[i0].pos[1], pts[i].pos[2] - pts[i0].pos[2]};
    T v = dot3(d, d);
    if (v > best) { best = v; i1 = i; }
  }
  used[i1] = true;
  keep.push_back(pts[i1]);
  int i2 = -1;
  best = -1;
  for (int i = 0; i < n; ++i) {
    if (used[i]) continue;
    T u[3], v[3], c[3];
    for (int k = 0; k < 3; ++k) { u[k] = pts[i1].pos[k] - pts[i0].pos[k]; v[k] = pts[i].pos[k] - pts[i0].pos[k]; }
    cross(u, v, c);
    T a = dot3(c, c);
    if (a > best) { best = a; i2 = i; }
  }
  used[i2] = true;
  keep.push_back(pts[i2]);
  int i3 = -1;
  best = -1;
  for (int i = 0; i < n; ++i) {
    if (used[i]) continue;
    // area added: max over the three triangle edges
    T add = 0;
    const int tri[3] = {i0, i1, i2};
    for (int e = 0; e < 3; ++e) {
      T u[3], v[3], c[3];
      for (int k = 0; k < 3; ++k) {
        u[k] = pts[tri[(e + 1) % 3]].pos[k] - pts[tri[e]].pos[k];
        v[k] = pts[i].pos[k] - pts[tri[e]].pos[k];
      }
      cross(u, v, c);
      add = std::max(add, dot3(c, c));
    }
    if (add > best) { best = add; i3 = i; }
  }
  keep.push_back(pts[i3]);
  pts.swap(keep);
}

// clip polygon (in 3D) by half-space n.x <= d
void clip_plane(std::vector<std::array<T, 3>>& poly, const T* n, T d) {
  std::vector<std::array<T, 3>> out;
  int m = (int)poly.size();
  for (int i = 0; i < m; ++i) {
    const auto& p = poly[i];
    const auto& q = poly[(i + 1) % m];
    T dp = n[0] * p[0] + n[1] * p[1] + n[2] * p[2] - d;
    T dq = n[0] * q[0] + n[1] * q[1] + n[2] * q[2] - d;
    if (dp <= 0) out.push_back(p);
    if ((dp < 0 && dq > 0) || (dp > 0 && dq < 0)) {
      T t = dp / (dp - dq);
      std::array<T, 3> x;
      for (int k = 0; k < 3; ++k) x[k] = p[k] + (q[k] - p[k]) * t;
      out.push_back(x);
    }
  }
  poly.swap(out);
}

// Face contact: reference box `ref` with outward unit normal nref (its face index `face`),
// incident box `inc`.  Produces points on the incident face inside the reference face, with
// dist = separation from the reference plane; `flip` makes the output normal point 1 -> 2.
void face_contact(const Geom& ref, int face, const T* nref, const Geom& inc, T margin, bool flip,
                  std::vector<Raw>& out) {
  // incident face: the face of inc whose outward normal is most anti-parallel to nref
  int best = 0;
  T bd = 0;
  for (int k = 0; k < 3; ++k) {
    T ax[3];
    axis(inc.mat, k, ax);
    T d = dot3(ax, nref);
    if (k == 0 || std::fabs(d) > std::fabs(bd)) { bd = d; best = k; }
  }
  T ninc[3];
  axis(inc.mat, best, ninc);
  T sgn = bd > 0 ? -1 : 1;          // outward normal of the incident face = sgn * axis
  T u[3], v[3], ctr[3];
  int k1 = (best + 1) % 3, k2 = (best + 2) % 3;
  axis(inc.mat, k1, u);
  axis(inc.mat, k2, v);
  for (int k = 0; k < 3; ++k) ctr[k] = inc.pos[k] + sgn * ninc[k] * inc.size[best];
  std::vector<std::array<T, 3>> poly(4);
  const T su[4] = {1, -1, -1, 1}, sv[4] = {1, 1, -1, -1};
  for (int i = 0; i < 4; ++i)
    for (int k = 0; k < 3; ++k) poly[i][k] = ctr[k] + su[i] * inc.size[k1] * u[k] + sv[i] * inc.size[k2] * v[k];
  // side planes of the reference face
  for (int j = 1; j <= 2; ++j) {
    int kk = (face + j) % 3;
    T ax[3];
    axis(ref.mat, kk, ax);
    T c = dot3(ax, ref.pos);
    clip_plane(poly, ax, c + ref.size[kk]);
    T nax[3] = {-ax[0], -ax[1], -ax[2]};
    clip_plane(poly, nax, -c + ref.size[kk]);
    if (poly.empty()) return;
  }
  T off = dot3(nref, ref.pos) + ref.size[face];
  std::vector<Raw> pts;
  for (const auto& q : poly) {
    T sep = nref[0] * q[0] + nref[1] * q[1] + nref[2] * q[2] - off;
    if (sep >= margin) continue;
    Raw r;
    for (int k = 0; k < 3; ++k) {
      r.pos[k] = q[k] - nref[k] * 0.5 * sep;
      r.normal[k] = flip ? -nref[k] : nref[k];
    }
    r.dist = sep;
    pts.push_back(r);
  }
  reduce4(pts);
  out.insert(out.end(), pts.begin(), pts.end());
}

void box_box(const Geom& g1, const Geom& g2, T margin, std::vector<Raw>& out) {
  T A[3][3], B[3][3], d[3];
  for (int k = 0; k < 3; ++k) { axis(g1.mat, k, A[k]); axis(g2.mat, k, B[k]); d[k] = g2.pos[k] - g1.pos[k]; }
  T best_face = 1e30, best_edge = 1e30;
  int face_axis = -1, edge_i = -1, edge_j = -1;
  T face_n[3] = {0, 0, 0}, edge_n[3] = {0, 0, 0};
  auto test = [&](const T* u, T& overlap, T* n) {
    T ra = 0, rb = 0;
    for (int k = 0; k < 3; ++k) { ra += g1.size[k] * std::fabs(dot3(u, A[k])); rb += g2.size[k] * std::fabs(dot3(u, B[k])); }
    T s = dot3(u, d);
    overlap = ra + rb - std::fabs(s);
    T sg = s >= 0 ? 1 : -1;
    for (int k = 0; k < 3; ++k) n[k] = sg * u[k];
  };
  for (int a = 0; a < 6; ++a) {
    const T* u = a < 3 ? A[a] : B[a - 3];
    T ov, n[3];
    test(u, ov, n);
    if (ov < -margin) return;
    if (ov < best_face) { best_face = ov; face_axis = a; for (int k = 0; k < 3; ++k) face_n[k] = n[k]; }
  }
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      T u[3];
      cross(A[i], B[j], u);
      T len = norm3(u);
      if (len < 1e-6) continue;
      for (int k = 0; k < 3; ++k) u[k] /= len;
      T ov, n[3];
      test(u, ov, n);
      if (ov < -margin) return;
      if (ov < best_edge) { best_edge = ov; edge_i = i; edge_j = j; for (int k = 0; k < 3; ++k) edge_n[k] = n[k]; }
    }
  if (edge_i >= 0 && best_edge < 0.95 * best_face - 1e-5) {
    // edge-edge: support edges of both boxes along the normal, closest points
    T p1[3], q1[3], p2[3], q2[3];
    T c1[3], c2[3];
    for (int k = 0; k < 3; ++k) { c1[k] = g1.pos[k]; c2[k] = g2.pos[k]; }
    for (int k = 0; k < 3; ++k) {
      if (k != edge_i) {
        T s = dot3(A[k], edge_n) >= 0 ? 1 : -1;
        for (int c = 0; c < 3; ++c) c1[c] += s * g1.size[k] * A[k][c];
      }
      if (k != edge_j) {
        T s = dot3(B[k], edge_n) >= 0 ? -1 : 1;
        for (int c = 0; c < 3; ++c) c2[c] += s * g2.size[k] * B[k][c];
      }
    }
    for (int c = 0; c < 3; ++c) {
      p1[c] = c1[c] - g1.size[edge_i] * A[edge_i][c]; q1[c] = c1[c] + g1.size[edge_i] * A[edge_i][c];
      p2[c] = c2[c] - g2.size[edge_j] * B[edge_j][c]; q2[c] = c2[c] + g2.size[edge_j] * B[edge_j][c];
    }
    T s, t;
    closest_segments(p1, q1, p2, q2, s, t);
    T x1[3], x2[3], pos[3];
    for (int c = 0; c < 3; ++c) {
      x1[c] = p1[c] + (q1[c] - p1[c]) * s;
      x2[c] = p2[c] + (q2[c] - p2[c]) * t;
      pos[c] = 0.5 * (x1[c] + x2[c]);
    }
    push(out, pos, edge_n, -best_edge);
    return;
  }
  if (face_axis < 3) {
    face_contact(g1, face_axis, face_n, g2, margin, false, out);
  } else {
    T nref[3] = {-face_n[0], -face_n[1], -face_n[2]};
    face_contact(g2, face_axis - 3, nref, g1, margin, true, out);
  }
}

// ------------------------------------------------------------------ dispatch
int narrowphase(const Geom& g1, const Geom& g2, T margin, std::vector<Raw>& out) {
  int t1 = g1.type, t2 = g2.type;
  if (t1 == PLANE) {
    if (t2 == SPHERE) plane_point(g1, g2.pos, g2.size[0], margin, out);
    else if (t2 == CAPSULE) {
      T a[3], b[3];
      segment(g2, a, b);
      plane_point(g1, a, g2.size[0], margin, out);
      plane_point(g1, b, g2.size[0], margin, out);
    } else if (t2 == BOX) plane_vertices(g1, box_corners(g2), margin, out);
    else if (t2 == MESH) plane_vertices(g1, mesh_world(g2), margin, out);
    return 1;
  }
  if (t1 == SPHERE && t2 == SPHERE) {
    T fb[3] = {0, 0, 1};
    sphere_sphere(g1.pos, g1.size[0], g2.pos, g2.size[0], margin, out, fb);
    return 1;
  }
  if (t1 == SPHERE && t2 == CAPSULE) {
    T a[3], b[3], s, t;
    segment(g2, a, b);
    closest_segments(g1.pos, g1.pos, a, b, s, t);
    T p[3], fb[3] = {0, 0, 1};
    for (int k = 0; k < 3; ++k) p[k] = a[k] + (b[k] - a[k]) * t;
    sphere_sphere(g1.pos, g1.size[0], p, g2.size[0], margin, out, fb);
    return 1;
  }
  if (t1 == SPHERE && t2 == BOX) { sphere_box(g1.pos, g1.size[0], g2, margin, out); return 1; }
  if (t1 == CAPSULE && t2 == CAPSULE) { capsule_capsule(g1, g2, margin, out); return 1; }
  if (t1 == CAPSULE && t2 == BOX) { capsule_box(g1, g2, margin, out); return 1; }
  if (t1 == BOX && t2 == BOX) { box_box(g1, g2, margin, out); return 1; }
  return 0;   // convex hull pairs: not yet supported
}

}  // namespace

void collision(const OrModel& m, World& w, const int32_t* body_active) {
  w.contacts.clear();
  w.overflow &= ~MX_OVERFLOW_NARROWPHASE;
  if ((m.opt_disableflags & 1) || (m.opt_disableflags & (1 << 4))) return;
  auto geom = [&](int g) {
    Geom x;
    x.id = g;
    x.type = m.geom_type[g];
    for (int k = 0; k < 3; ++k) { x.pos[k] = w.geom_xpos[3 * g + k]; x.size[k] = m.geom_size[3 * g + k]; }
    for (int k = 0; k < 9; ++k) x.mat[k] = w.geom_xmat[9 * g + k];
    if (x.type == MESH) {
      int id = m.geom_dataid[g];
      x.vert = m.mesh_vert + 3 * m.mesh_vertadr[id];
      x.nvert = m.mesh_vertnum[id];
    }
    return x;
  };
  for (int p = 0; p < m.npair; ++p) {
    int g1 = m.pair_geom[2 * p], g2 = m.pair_geom[2 * p + 1];
    if (body_active && (!body_active[m.geom_body[g1]] || !body_active[m.geom_body[g2]])) continue;
    T margin = std::max(m.geom_margin[g1], m.geom_margin[g2]);
    T gap = std::max(m.geom_gap[g1], m.geom_gap[g2]);
    // broadphase: plane half-space or bounding spheres
    const T* c1 = &w.geom_xpos[3 * g1];
    const T* c2 = &w.geom_xpos[3 * g2];
    if (m.geom_type[g1] == PLANE) {
      T n[3] = {w.geom_xmat[9 * g1 + 2], w.geom_xmat[9 * g1 + 5], w.geom_xmat[9 * g1 + 8]};
      T d[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
      if (dot3(n, d) - m.geom_rbound[g2] > margin) continue;
    } else {
      T d[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
      if (norm3(d) > m.geom_rbound[g1] + m.geom_rbound[g2] + margin) continue;
    }
    std::vector<Raw> raw;
    narrowphase(geom(g1), geom(g2), margin, raw);
    // material (contact_material, mjwarp_contact.cuh:56-101)
    int pr1 = m.geom_priority[g1], pr2 = m.geom_priority[g2];
    int dim;
    T fr[3], solref[2], solimp[5];
    if (pr1 != pr2) {
      int g = pr1 > pr2 ? g1 : g2;
      dim = m.geom_condim[g];
      for (int k = 0; k < 3; ++k) fr[k] = m.geom_friction[3 * g + k];
      for (int k = 0; k < 2; ++k) solref[k] = m.geom_solref[2 * g + k];
      for (int k = 0; k < 5; ++k) solimp[k] = m.geom_solimp[5 * g + k];
    } else {
      dim = std::max(m.geom_condim[g1], m.geom_condim[g2]);
      for (int k = 0; k < 3; ++k) fr[k] = std::max(m.geom_friction[3 * g1 + k], m.geom_friction[3 * g2 + k]);
      T s1 = m.geom_solmix[g1], s2 = m.geom_solmix[g2], mix;
      if (s1 < kMinVal && s2 < kMinVal) mix = 0.5;
      else if (s1 < kMinVal) mix = 0;
      else if (s2 < kMinVal) mix = 1;
      else mix = s1 / (s1 + s2);
      if (m.geom_solref[2 * g1] > 0 && m.geom_solref[2 * g2] > 0)
        for (int k = 0; k < 2; ++k) solref[k] = mix * m.geom_solref[2 * g1 + k] + (1 - mix) * m.geom_solref[2 * g2 + k];
      else
        for (int k = 0; k < 2; ++k) solref[k] = std::min(m.geom_solref[2 * g1 + k], m.geom_solref[2 * g2 + k]);
      for (int k = 0; k < 5; ++k) solimp[k] = mix * m.geom_solimp[5 * g1 + k] + (1 - mix) * m.geom_solimp[5 * g2 + k];
    }
    for (const Raw& r : raw) {
      if ((int)w.contacts.size() >= m.nconmax) { w.overflow |= MX_OVERFLOW_NARROWPHASE; break; }
      Contact c;
      for (int k = 0; k < 3; ++k) c.pos[k] = r.pos[k];
      make_frame(r.normal, c.frame);
      c.dist = r.dist;
      c.friction[0] = fr[0]; c.friction[1] = fr[0]; c.friction[2] = fr[1]; c.friction[3] = fr[2]; c.friction[4] = fr[2];
      for (int k = 0; k < 2; ++k) c.solref[k] = solref[k];
      for (int k = 0; k < 5; ++k) c.solimp[k] = solimp[k];
      c.includemargin = margin - gap;
      c.geom[0] = g1; c.geom[1] = g2;
      c.dim = dim;
      c.efc_address = -1;
      w.contacts.push_back(c);
    }
  }
}

}  // namespace orc
