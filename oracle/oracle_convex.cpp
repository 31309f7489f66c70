// Convex collision of the CPU FP64 oracle -- TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// Restates, in double, the reference's rigid CCD for convex pair families:
//   support functions        gpu/cuda/collision/mjwarp_convex_geometry.cuh:17-68
//   signed-volume distance   gpu/cuda/collision/mjwarp_convex_simplex.cuh:13-79
//   GJK with cutoff          gpu/cuda/collision/mjwarp_convex_gjk.cuh:21-88
//   GJK phase and EPA        gpu/cuda/collision/mjwarp_convex_epa.cuh:18-261
//   box-box manifold         gpu/cuda/collision/mjwarp_box_manifold.cuh:7-133
//   pair driver              gpu/cuda/collision/mjwarp_convex_collision.cuh:43-79
// Hull support scans every vertex (the reference hill-climbs the hull graph for hulls of 10 or
// more vertices; both return the support maximizer and differ only on exact ties).  The MPR section
// restates libccd (BSD licence; its notice is reproduced there).
#include "oracle_geom.h"

namespace orc {
inline namespace narrow {
namespace {

struct V {
  T v[3];
  T& operator[](int i) { return v[i]; }
  T operator[](int i) const { return v[i]; }
};
V mk(T x, T y, T z) { V r; r.v[0] = x; r.v[1] = y; r.v[2] = z; return r; }
V ld(const T* p) { return mk(p[0], p[1], p[2]); }
V operator+(V a, V b) { return mk(a[0] + b[0], a[1] + b[1], a[2] + b[2]); }
V operator-(V a, V b) { return mk(a[0] - b[0], a[1] - b[1], a[2] - b[2]); }
V operator-(V a) { return mk(-a[0], -a[1], -a[2]); }
V operator*(V a, T s) { return mk(a[0] * s, a[1] * s, a[2] * s); }
V operator*(T s, V a) { return a * s; }
T dot(V a, V b) { return a[0] * b[0] + a[1] * b[1] + a[2] * b[2]; }
V crs(V a, V b) { return mk(a[1] * b[2] - a[2] * b[1], a[2] * b[0] - a[0] * b[2], a[0] * b[1] - a[1] * b[0]); }
V unit(V a) { T n = std::sqrt(dot(a, a)); return n > 0 ? a * (1 / n) : mk(0, 0, 0); }
V divv(V a, T s) { return mk(a[0] / s, a[1] / s, a[2] / s); }
V rot(const T* R, V x) { return mk(R[0] * x[0] + R[1] * x[1] + R[2] * x[2], R[3] * x[0] + R[4] * x[1] + R[5] * x[2],
                                   R[6] * x[0] + R[7] * x[1] + R[8] * x[2]); }
V rotT(const T* R, V x) { return mk(R[0] * x[0] + R[3] * x[1] + R[6] * x[2], R[1] * x[0] + R[4] * x[1] + R[7] * x[2],
                                    R[2] * x[0] + R[5] * x[1] + R[8] * x[2]); }
T sgn(T x) { return x > 0 ? 1 : x < 0 ? -1 : 0; }

constexpr T kFloatMax = 1e30, kConvexMin = 1e-15;

// ------------------------------------------------------------------ support
struct CGeom {
  V pos, size;
  const T* rot;
  const T* vert;     // hull vertices in the geom frame
  int nvert, cached;  // cached: hull vertex of the last support query (-1: none)
  T margin;
};
struct Support { V point; int cached, vertex; };

// Support point of geom g (type) in the world direction d, inflated by half the margin.
Support support(const CGeom& g, int type, V d) {
  Support s{mk(0, 0, 0), -1, -1};
  if (type == SPHERE) { s.point = g.pos + (g.size[0] + 0.5 * g.margin) * d; return s; }
  V local = rotT(g.rot, d), res = mk(0, 0, 0);
  if (type == BOX) {
    // a zero component picks the negative corner, so bit k of the vertex index is +size
    V sign = mk(local[0] > 0 ? 1 : -1, local[1] > 0 ? 1 : -1, local[2] > 0 ? 1 : -1);
    for (int k = 0; k < 3; ++k) res[k] = sign[k] * g.size[k];
    s.point = rot(g.rot, res) + g.pos;
    s.vertex = int(sign[0] > 0) + 2 * int(sign[1] > 0) + 4 * int(sign[2] > 0);
  } else if (type == CAPSULE) {
    res = local * g.size[0];
    res[2] += sgn(local[2]) * g.size[1];
    s.point = rot(g.rot, res) + g.pos;
  } else if (type == MESH) {
    T best = -1e30;
    if (g.cached > -1) { s.cached = g.cached; s.point = ld(g.vert + 3 * g.cached); best = dot(s.point, local); }
    for (int i = 0; i < g.nvert; ++i) {
      V v = ld(g.vert + 3 * i);
      T h = dot(v, local);
      if (h > best) { best = h; s.point = v; s.cached = i; }
    }
    s.vertex = s.cached;
    s.point = rot(g.rot, s.point) + g.pos;
  }
  if (g.margin > 0) s.point = s.point + d * (0.5 * g.margin);
  return s;
}

// ------------------------------------------------------------------ signed-volume distance
struct W4 { T w[4]; T& operator[](int k) { return w[k]; } T operator[](int k) const { return w[k]; } };
W4 w4(T a, T b, T c, T d) { W4 r; r.w[0] = a; r.w[1] = b; r.w[2] = c; r.w[3] = d; return r; }

bool same_sign(T a, T b) { return (a > 0 && b > 0) || (a < 0 && b < 0); }

V origin_on_line(V a, V b) {
  V d = b - a;
  T s = -dot(b, d) / dot(d, d);
  return b + s * d;
}

V origin_on_plane(V a, V b, V c, bool& degenerate) {
  V d21 = b - a, d31 = c - a, d32 = c - b;
  degenerate = false;
  V n = crs(d32, d21);
  T nv = dot(n, b), nn = dot(n, n);
  if (nn == 0) { degenerate = true; return mk(0, 0, 0); }
  if (nv != 0 && nn > kConvexMin) return (nv / nn) * n;
  n = crs(d21, d31);
  nv = dot(n, a); nn = dot(n, n);
  if (nn == 0) { degenerate = true; return mk(0, 0, 0); }
  if (nv != 0 && nn > kConvexMin) return (nv / nn) * n;
  n = crs(d31, d32);
  nv = dot(n, c); nn = dot(n, n);
  return (nv / nn) * n;
}

W4 simplex1(V a, V b) {   // segment
  V p = origin_on_line(a, b);
  T mx = a[0] - b[0];
  int idx = 0;
  for (int k = 1; k < 3; ++k) { T v = a[k] - b[k]; if (std::fabs(v) >= std::fabs(mx)) { mx = v; idx = k; } }
  T c1 = p[idx] - b[idx], c2 = a[idx] - p[idx];
  if (same_sign(mx, c1) && same_sign(mx, c2)) return w4(c1 / mx, c2 / mx, 0, 0);
  return w4(0, 1, 0, 0);
}

T minor2(V a, V b, V c, int i, int j) { V u = b - a, v = c - a; return u[i] * v[j] - u[j] * v[i]; }
T area2(V p, V a, V b, int i, int j) { V u = a - p, v = b - p; return u[i] * v[j] - u[j] * v[i]; }

W4 simplex2(V a, V b, V c) {   // triangle
  bool deg;
  V p = origin_on_plane(a, b, c, deg);
  if (deg) return simplex1(a, b);
  T m14 = minor2(a, b, c, 1, 2), m24 = minor2(a, b, c, 0, 2), m34 = minor2(a, b, c, 0, 1), mx;
  int i, j;
  if (std::fabs(m14) >= std::fabs(m24) && std::fabs(m14) >= std::fabs(m34)) { mx = m14; i = 1; j = 2; }
  else if (std::fabs(m24) >= std::fabs(m34)) { mx = m24; i = 0; j = 2; }
  else { mx = m34; i = 0; j = 1; }
  T c31 = area2(p, b, c, i, j), c32 = area2(p, c, a, i, j), c33 = area2(p, a, b, i, j);
  bool k1 = same_sign(mx, c31), k2 = same_sign(mx, c32), k3 = same_sign(mx, c33);
  if (k1 && k2 && k3) return w4(c31 / mx, c32 / mx, c33 / mx, 0);
  W4 w = w4(0, 0, 0, 0);
  T best = kFloatMax;
  if (!k1) { W4 s = simplex1(b, c); V x = s[0] * b + s[1] * c; w = w4(0, s[0], s[1], 0); best = dot(x, x); }
  if (!k2) { W4 s = simplex1(a, c); V x = s[0] * a + s[1] * c; T d = dot(x, x); if (d < best) { w = w4(s[0], 0, s[1], 0); best = d; } }
  if (!k3) { W4 s = simplex1(a, b); V x = s[0] * a + s[1] * b; T d = dot(x, x); if (d < best) w = w4(s[0], s[1], 0, 0); }
  return w;
}

T det3(V a, V b, V c) { return dot(a, crs(b, c)); }

W4 simplex3(V a, V b, V c, V d) {   // tetrahedron
  T c41 = -det3(b, c, d), c42 = det3(a, c, d), c43 = -det3(a, b, d), c44 = det3(a, b, c);
  T det = c41 + c42 + c43 + c44;
  bool k1 = same_sign(det, c41), k2 = same_sign(det, c42), k3 = same_sign(det, c43), k4 = same_sign(det, c44);
  if (k1 && k2 && k3 && k4) return w4(c41 / det, c42 / det, c43 / det, c44 / det);
  W4 w = w4(0, 0, 0, 0);
  T best = kFloatMax;
  if (!k1) { W4 s = simplex2(b, c, d); V x = s[0] * b + s[1] * c + s[2] * d; w = w4(0, s[0], s[1], s[2]); best = dot(x, x); }
  if (!k2) { W4 s = simplex2(a, c, d); V x = s[0] * a + s[1] * c + s[2] * d; T e = dot(x, x); if (e < best) { w = w4(s[0], 0, s[1], s[2]); best = e; } }
  if (!k3) { W4 s = simplex2(a, b, d); V x = s[0] * a + s[1] * b + s[2] * d; T e = dot(x, x); if (e < best) { w = w4(s[0], s[1], 0, s[2]); best = e; } }
  if (!k4) { W4 s = simplex2(a, b, c); V x = s[0] * a + s[1] * b + s[2] * c; T e = dot(x, x); if (e < best) w = w4(s[0], s[1], s[2], 0); }
  return w;
}

W4 simplex_weights(int n, const V* s) {
  if (n == 4) return simplex3(s[0], s[1], s[2], s[3]);
  if (n == 3) return simplex2(s[0], s[1], s[2]);
  if (n == 2) return simplex1(s[0], s[1]);
  return w4(1, 0, 0, 0);
}

V combine(int n, const W4& w, const V* s) {
  V x = w[0] * s[0];
  for (int k = 1; k < n; ++k) x = x + w[k] * s[k];
  return x;
}

// ------------------------------------------------------------------ GJK
struct Gjk {
  bool separated;
  T dist;
  V x1, x2;
  int dim;
  V s[4], s1[4], s2[4];
  int v1[4], v2[4], index1, index2;
};

Gjk gjk(T tol, int maxit, CGeom g1, CGeom g2, V init1, V init2, int t1, int t2, T cutoff, bool discrete) {
  V s[4], s1[4], s2[4];
  int v1[4] = {0, 0, 0, 0}, v2[4] = {0, 0, 0, 0}, n = 0;
  for (int k = 0; k < 4; ++k) s[k] = s1[k] = s2[k] = mk(0, 0, 0);
  W4 w = w4(1, 0, 0, 0);
  T eps = discrete ? 0 : 0.5 * tol * tol, min_norm = discrete ? kConvexMin : tol;
  V x = init1 - init2;
  T norm = std::sqrt(dot(x, x)), prev = 0;
  for (int it = 0; it < maxit; ++it) {
    if (norm < min_norm || std::fabs(prev - norm) < kConvexMin) break;
    V dir = divv(x, norm);
    if (discrete && norm < 1e-4) {
      // near contact, tune the search direction to the current simplex feature
      if (n == 2) {
        V e = s[1] - s[0];
        T l2 = dot(e, e);
        if (l2 > 1e-30) {
          dir = dir - (dot(dir, e) / l2) * e;
          T l = std::sqrt(dot(dir, dir));
          if (l > kConvexMin) dir = divv(dir, l);
        }
      } else if (n == 3) {
        V nn = crs(s[1] - s[0], s[2] - s[0]);
        T l = std::sqrt(dot(nn, nn));
        if (l > kConvexMin) dir = divv(sgn(dot(dir, nn)) * nn, l);
      }
    }
    Support a = support(g1, t1, -dir), b = support(g2, t2, dir);
    s1[n] = a.point; g1.cached = a.cached; v1[n] = a.vertex;
    s2[n] = b.point; g2.cached = b.cached; v2[n] = b.vertex;
    s[n] = s1[n] - s2[n];
    if (dot(x, x - s[n]) < eps) break;
    T lower = dot(x, s[n]);
    bool cut = (cutoff == 0 && lower > 0) || (cutoff != 0 && cutoff < kFloatMax && lower > 0 && lower >= cutoff * norm);
    if (cut && discrete && norm < 1e-4 && (n == 2 || n == 3)) {
      // the tuned direction is the one the support plane certifies
      lower = dot(dir, s[n]);
      T cn = std::sqrt(dot(dir, dir));
      cut = cn > kConvexMin && lower > 0 && (cutoff == 0 || (cutoff < kFloatMax && lower >= cutoff * cn));
    }
    if (cut) {
      Gjk r{};
      r.separated = true; r.dim = 0; r.dist = kFloatMax; r.index1 = g1.cached; r.index2 = g2.cached;
      return r;
    }
    w = simplex_weights(n + 1, s);
    n = 0;
    for (int i = 0; i < 4; ++i) {
      if (w[i] == 0) continue;
      s[n] = s[i]; s1[n] = s1[i]; s2[n] = s2[i]; v1[n] = v1[i]; v2[n] = v2[i]; w[n] = w[i];
      ++n;
    }
    if (n < 1) break;
    x = combine(n, w, s);
    prev = norm;
    norm = std::sqrt(dot(x, x));
    if (n == 4) break;
  }
  Gjk r{};
  r.separated = false;
  r.x1 = n == 0 ? init1 : combine(n, w, s1);
  r.x2 = n == 0 ? init2 : combine(n, w, s2);
  if (norm > 0) {
    V dir = divv(x, norm);
    Support a = support(g1, t1, -dir), b = support(g2, t2, dir);
    r.separated = dot(x, a.point - b.point) > 0;
  }
  r.dist = n == 4 && !r.separated ? 0 : norm;
  r.dim = n;
  for (int i = 0; i < 4; ++i) { r.s[i] = s[i]; r.s1[i] = s1[i]; r.s2[i] = s2[i]; r.v1[i] = v1[i]; r.v2[i] = v2[i]; }
  r.index1 = g1.cached; r.index2 = g2.cached;
  return r;
}

bool discrete_pair(int a, int b) { return (a == BOX || a == MESH) && (b == BOX || b == MESH); }

struct Phase {
  bool needs_epa;
  T distance;
  V x1, x2;
  Gjk r;
  CGeom g1, g2;
  bool require_enclosing;
};

// Spheres and capsules are shrunk to their core (point / segment) for the first GJK and the radii
// added back; deep penetration retries with the full shapes.  Box pairs whose GJK stalls above the
// tolerance retry once from the current witnesses and then go to EPA with an enclosure check.
Phase gjk_phase(T tol, T cutoff, int iters, CGeom a, CGeom b, int t1, int t2, V init1, V init2) {
  V size1 = a.size, size2 = b.size;
  T m1 = a.margin, m2 = b.margin, full1 = 0, full2 = 0, r1 = 0, r2 = 0;
  bool discrete = discrete_pair(t1, t2) && m1 == 0 && m2 == 0;
  if (t1 == SPHERE || t1 == CAPSULE) { r1 = a.size[0]; full1 = r1 + 0.5 * m1; a.margin = 0; a.size[0] = 0; }
  if (t2 == SPHERE || t2 == CAPSULE) { r2 = b.size[0]; full2 = r2 + 0.5 * m2; b.margin = 0; b.size[0] = 0; }
  if (r1 + r2 > 0) {
    cutoff += full1 + full2;
    Gjk r = gjk(tol, iters, a, b, init1, init2, t1, t2, cutoff, discrete);
    a.cached = r.index1; b.cached = r.index2;
    if (r.dist > tol) {
      if (r.dist == kFloatMax) return Phase{false, r.dist, r.x1, r.x2, Gjk{}, a, b, false};
      V n = unit(r.x2 - r.x1), x1 = r.x1, x2 = r.x2;
      if (full1 > 0) x1 = x1 + full1 * n;
      if (full2 > 0) x2 = x2 - full2 * n;
      a.size = size1; a.margin = m1; b.size = size2; b.margin = m2;
      return Phase{false, r.dist - (full1 + full2), x1, x2, r, a, b, false};
    }
    a.size = size1; a.margin = m1; b.size = size2; b.margin = m2;
    cutoff -= full1 + full2;
  }
  Gjk r = gjk(tol, iters, a, b, init1, init2, t1, t2, cutoff, discrete);
  a.cached = r.index1; b.cached = r.index2;
  bool retry_box = t1 == BOX && t2 == BOX && discrete && r.dist > tol && r.dim >= 2 && !r.separated;
  if (retry_box) {
    Gjk q = gjk(tol, iters, a, b, r.x1, r.x2, t1, t2, cutoff, discrete);
    if (q.separated || (q.dim >= 2 && q.dist < r.dist)) r = q;
    a.cached = r.index1; b.cached = r.index2;
  }
  if ((r.dist > tol && !retry_box) || r.dim < 2 || r.separated) return Phase{false, r.dist, r.x1, r.x2, Gjk{}, a, b, false};
  return Phase{true, r.dist, r.x1, r.x2, r, a, b, retry_box};
}

// ------------------------------------------------------------------ EPA
struct Polytope {
  std::vector<V> vert;          // 2 per polytope vertex: support point on geom 1, on geom 2
  std::vector<int> vidx;        // 2 per polytope vertex: feature index on geom 1, on geom 2
  std::vector<int> face;        // packed a | b << 10 | c << 20; bit 31 deleted, bit 30 invalid
  std::vector<V> proj;          // closest point of each face plane to the origin
  std::vector<T> norm2;
  std::vector<int> horizon;
  int face_capacity, horizon_capacity, status = 0, nvert = 0, nface = 0, nhorizon = 0;
  V center;
  Polytope(int vcap, int fcap, int hcap)
      : vert(2 * vcap), vidx(2 * vcap), face(fcap), proj(fcap), norm2(fcap), horizon(hcap),
        face_capacity(fcap), horizon_capacity(hcap), center(mk(0, 0, 0)) {}
  V vertex(int i) const { return vert[2 * i] - vert[2 * i + 1]; }
};

struct Epa { T distance; int ncontact; V x1, x2; int face; bool horizon_overflow = false; };

V triangle_affine(V a, V b, V c, V p) {
  T m14 = minor2(a, b, c, 1, 2), m24 = minor2(a, b, c, 0, 2), m34 = minor2(a, b, c, 0, 1), mx;
  int i, j;
  if (std::fabs(m14) >= std::fabs(m24) && std::fabs(m14) >= std::fabs(m34)) { mx = m14; i = 1; j = 2; }
  else if (std::fabs(m24) >= std::fabs(m34)) { mx = m24; i = 0; j = 2; }
  else { mx = m34; i = 0; j = 1; }
  return mk(area2(p, b, c, i, j) / mx, area2(p, c, a, i, j) / mx, area2(p, a, b, i, j) / mx);
}

bool triangle_contains(V a, V b, V c, V p) {
  V w = triangle_affine(a, b, c, p);
  if (w[0] < 0 || w[1] < 0 || w[2] < 0) return false;
  V d = w[0] * a + w[1] * b + w[2] * c - p;
  return std::sqrt(dot(d, d)) < kConvexMin;
}

bool same_side(V a, V b, V c, V d) {
  V n = crs(b - a, c - a);
  T one = dot(n, d - a), two = dot(n, -a);
  return (one > 0 && two > 0) || (one < 0 && two < 0);
}

bool tetra_contains_origin(V a, V b, V c, V d) {
  return same_side(a, b, c, d) && same_side(b, c, d, a) && same_side(c, d, a, b) && same_side(d, a, b, c);
}

T attach_face(Polytope& p, int index, int a, int b, int c) {
  if (p.nface == p.face_capacity) return 0;
  V one = p.vertex(a), two = p.vertex(b), three = p.vertex(c);
  bool bad;
  V r = origin_on_plane(three, two, one, bad);
  if (bad) return 0;
  if (dot(r, one - p.center) < 0) r = -r;
  p.face[index] = a + (b << 10) + (c << 20);
  p.proj[index] = r;
  p.norm2[index] = dot(r, r);
  return p.norm2[index];
}

void epa_support(Polytope& p, int index, const CGeom& a, const CGeom& b, int t1, int t2, V d, int& c1, int& c2) {
  Support one = support(a, t1, d), two = support(b, t2, -d);
  p.vert[2 * index] = one.point; p.vert[2 * index + 1] = two.point;
  p.vidx[2 * index] = one.vertex; p.vidx[2 * index + 1] = two.vertex;
  c1 = one.cached; c2 = two.cached;
}

void initial_vertices(Polytope& p, const Gjk& r, int n) {
  for (int i = 0; i < n; ++i) {
    p.vert[2 * i] = r.s1[i]; p.vert[2 * i + 1] = r.s2[i];
    p.vidx[2 * i] = r.v1[i]; p.vidx[2 * i + 1] = r.v2[i];
  }
}

void replace_triangle(const Polytope& p, Gjk& r, int a, int b, int c) {
  int idx[3] = {a, b, c};
  for (int i = 0; i < 3; ++i) {
    int j = idx[i];
    r.s1[i] = p.vert[2 * j]; r.s2[i] = p.vert[2 * j + 1]; r.s[i] = r.s1[i] - r.s2[i];
    r.v1[i] = p.vidx[2 * j]; r.v2[i] = p.vidx[2 * j + 1];
  }
  r.dim = 3;
}

// Segment simplex: a triangular bipyramid around it (three supports 120 degrees apart).
void polytope_segment(Polytope& p, Gjk& r, const CGeom& a, const CGeom& b, int t1, int t2) {
  V diff = r.s[1] - r.s[0];
  p.center = 0.5 * (r.s[0] + r.s[1]);
  int index = 0;
  T value = kFloatMax;
  for (int i = 0; i < 3; ++i) if (std::fabs(diff[i]) < value) { value = std::fabs(diff[i]); index = i; }
  V ax = mk(0, 0, 0);
  ax[index] = 1;
  V d1 = crs(ax, diff), u = divv(diff, std::sqrt(dot(diff, diff)));
  // rotation by 120 degrees about u: -1/2 I + 3/2 u u^T + (sqrt(3)/2) [u]x
  const T s3 = 0.86602540378;
  T R[9];
  for (int i = 0; i < 3; ++i) for (int j = 0; j < 3; ++j) R[3 * i + j] = (i == j ? -0.5 : 0) + 1.5 * u[i] * u[j];
  R[1] -= u[2] * s3; R[2] += u[1] * s3; R[3] += u[2] * s3; R[5] -= u[0] * s3; R[6] -= u[1] * s3; R[7] += u[0] * s3;
  V dirs[3];
  dirs[0] = d1; dirs[1] = rot(R, d1); dirs[2] = rot(R, dirs[1]);
  initial_vertices(p, r, 2);
  int c1, c2;
  for (int i = 0; i < 3; ++i) epa_support(p, i + 2, a, b, t1, t2, divv(dirs[i], std::sqrt(dot(dirs[i], dirs[i]))), c1, c2);
  const int faces[6][3] = {{0, 2, 3}, {0, 4, 2}, {0, 3, 4}, {1, 3, 2}, {1, 2, 4}, {1, 4, 3}};
  for (int i = 0; i < 6; ++i)
    if (attach_face(p, i, faces[i][0], faces[i][1], faces[i][2]) < 1e-10) {
      p.status = -1;
      replace_triangle(p, r, faces[i][0], faces[i][1], faces[i][2]);
      return;
    }
  V v2 = p.vertex(2), v3 = p.vertex(3), v4 = p.vertex(4), v1 = r.s[0], base = r.s[1] - v1;
  T one = det3(v2 - v1, v3 - v1, base), two = det3(v3 - v1, v4 - v1, base), three = det3(v4 - v1, v2 - v1, base);
  if (!((one >= 0 && two >= 0 && three >= 0) || (one <= 0 && two <= 0 && three <= 0))) { p.status = 1; return; }
  p.nvert = 5; p.nface = 6; p.status = 0;
}

// Triangle simplex: a bipyramid with supports along both triangle normals.
void polytope_triangle(Polytope& p, Gjk& r, const CGeom& a, const CGeom& b, int t1, int t2, bool& require_enclosing) {
  p.center = (r.s[0] + r.s[1] + r.s[2]) * (1.0 / 3.0);
  V n = crs(r.s[1] - r.s[0], r.s[2] - r.s[0]);
  T norm = std::sqrt(dot(n, n));
  if (norm < kConvexMin) { p.status = 2; return; }
  n = divv(n, norm);
  initial_vertices(p, r, 3);
  int c1, c2;
  epa_support(p, 3, a, b, t1, t2, -n, c1, c2);
  epa_support(p, 4, a, b, t1, t2, n, c1, c2);
  V v1 = r.s[0], v2 = r.s[1], v3 = r.s[2], v4 = p.vertex(3), v5 = p.vertex(4);
  if (triangle_contains(v1, v2, v3, v4)) { p.status = 3; return; }
  if (triangle_contains(v1, v2, v3, v5)) { p.status = 4; return; }
  if (r.dist > 1e-5 && !tetra_contains_origin(v1, v2, v3, v4) && !tetra_contains_origin(v1, v2, v3, v5)) { p.status = 5; return; }
  const int faces[6][3] = {{4, 0, 1}, {4, 2, 0}, {4, 1, 2}, {3, 1, 0}, {3, 0, 2}, {3, 2, 1}};
  bool box = t1 == BOX && t2 == BOX && a.margin == 0 && b.margin == 0;
  for (int i = 0; i < 6; ++i) {
    T d2 = attach_face(p, i, faces[i][0], faces[i][1], faces[i][2]);
    if (require_enclosing || box) {
      if (!(d2 > 0)) { p.status = 6 + i; return; }
      if (d2 < 1e-10) require_enclosing = true;
    } else if (d2 < 1e-10) { p.status = 6 + i; return; }
  }
  p.nvert = 5; p.nface = 6; p.status = 0;
}

void polytope_tetrahedron(Polytope& p, Gjk& r) {
  p.center = 0.25 * (r.s[0] + r.s[1] + r.s[2] + r.s[3]);
  initial_vertices(p, r, 4);
  T dist[4];
  int closest = 0;
  const int faces[4][3] = {{0, 1, 2}, {0, 3, 1}, {0, 2, 3}, {3, 2, 1}};
  for (int i = 0; i < 4; ++i) {
    dist[i] = attach_face(p, i, faces[i][0], faces[i][1], faces[i][2]);
    if (dist[i] < 1e-17) { p.status = -1; replace_triangle(p, r, faces[i][0], faces[i][1], faces[i][2]); return; }
    if (i == 1) closest = dist[0] < dist[1] ? 0 : 1;
    else if (i > 1 && dist[i] < dist[closest]) closest = i;
  }
  if (!tetra_contains_origin(r.s[0], r.s[1], r.s[2], r.s[3])) {
    if (dist[closest] > kConvexMin) { p.status = 12; return; }
    p.status = -1;
    replace_triangle(p, r, faces[closest][0], faces[closest][1], faces[closest][2]);
    return;
  }
  p.nvert = 4; p.nface = 4; p.status = 0;
}

// Horizon edge set: an edge seen twice is interior and removed (swap with the last).
int add_edge(Polytope& p, int a, int b) {
  int n = p.nhorizon;
  if (n < 0) return -1;
  int edge = (std::min(a, b) << 10) | std::max(a, b);
  for (int i = 0; i < n; ++i)
    if (edge == p.horizon[i]) { p.horizon[i] = p.horizon[n - 1]; return n - 1; }
  if (n == p.horizon_capacity) return -1;
  p.horizon[n] = edge;
  return n + 1;
}

void face_edges(Polytope& p, int face) {
  int a = face & 0x3ff, b = (face >> 10) & 0x3ff, c = (face >> 20) & 0x3ff;
  p.nhorizon = add_edge(p, a, b);
  p.nhorizon = add_edge(p, b, c);
  p.nhorizon = add_edge(p, c, a);
}

bool deleted(int f) { return (unsigned(f) & 0x80000000u) != 0; }
bool invalid(int f) { return (unsigned(f) & 0xc0000000u) != 0; }
int mark(int f, unsigned bit) { return int(unsigned(f) | bit); }

Epa witness(const Polytope& p, int face) {
  int packed = p.face[face], a = packed & 0x3ff, b = (packed >> 10) & 0x3ff, c = (packed >> 20) & 0x3ff;
  V w = triangle_affine(p.vertex(a), p.vertex(b), p.vertex(c), p.proj[face]);
  V x1 = w[0] * p.vert[2 * a] + w[1] * p.vert[2 * b] + w[2] * p.vert[2 * c];
  V x2 = w[0] * p.vert[2 * a + 1] + w[1] * p.vert[2 * b + 1] + w[2] * p.vert[2 * c + 1];
  return Epa{-std::sqrt(p.norm2[face]), 1, x1, x2, face};
}

Epa epa_expand(T tol, int iters, Polytope& p, CGeom a, CGeom b, int t1, int t2, bool discrete) {
  T upper = kFloatMax, upper2 = kFloatMax, eps = discrete ? 1e-7 : tol;
  int index = -1, nvalid = p.nface;
  iters = std::min(iters, 1000);
  for (int it = 0; it < iters; ++it) {
    int prev = index;
    index = -1;
    T lower2 = kFloatMax;
    for (int i = 0; i < p.nface; ++i)
      if (!invalid(p.face[i]) && p.norm2[i] < lower2) { index = i; lower2 = p.norm2[i]; }
    if (lower2 > upper2 || index < 0) { index = prev; break; }
    if (lower2 <= 0) break;
    T lower = std::sqrt(lower2);
    int wi = p.nvert, c1, c2;
    V pr = p.proj[index];
    epa_support(p, wi, a, b, t1, t2, divv(pr, lower), c1, c2);
    V w = p.vertex(wi);
    a.cached = c1; b.cached = c2;
    ++p.nvert;
    T next = dot(pr, w) / lower;
    if (next < upper) { upper = next; upper2 = upper * upper; }
    if (upper - lower < eps) break;
    if (discrete) {
      bool repeated = false;
      for (int i = 0; i < p.nvert - 1; ++i)
        if (p.vidx[2 * i] == p.vidx[2 * wi] && p.vidx[2 * i + 1] == p.vidx[2 * wi + 1]) { repeated = true; break; }
      if (repeated) break;
    }
    --nvalid;
    p.face[index] = mark(p.face[index], 0x80000000u);
    face_edges(p, p.face[index]);
    if (p.nhorizon == -1) { index = -1; break; }
    for (int i = 0; i < p.nface; ++i) {
      if (deleted(p.face[i])) continue;
      if (dot(p.proj[i], w) - p.norm2[i] > 1e-10) {
        if (!invalid(p.face[i])) --nvalid;
        p.face[i] = mark(p.face[i], 0x80000000u);
        face_edges(p, p.face[i]);
        if (p.nhorizon == -1) { index = -1; break; }
      }
    }
    if (index == -1) break;
    for (int i = 0; i < p.nhorizon; ++i) {
      int e = p.horizon[i];
      T d2 = attach_face(p, p.nface, wi, e & 0x3ff, (e >> 10) & 0x3ff);
      if (d2 == 0) { index = -1; break; }
      ++p.nface;
      if (d2 >= lower2 && d2 <= upper2) ++nvalid;
      else p.face[p.nface - 1] = mark(p.face[p.nface - 1], 0x40000000u);
    }
    if (nvalid == 0 || index == -1) break;
    p.nhorizon = 0;
  }
  if (index >= 0) return witness(p, index);
  Epa none{kFloatMax, 0, mk(0, 0, 0), mk(0, 0, 0), -1};
  none.horizon_overflow = p.nhorizon == -1;
  return none;
}

bool multicontact_supported(const CGeom& a, const CGeom& b, int t1, int t2) {
  if (a.margin != 0 || b.margin != 0) return false;
  bool f1 = t1 == BOX || t1 == MESH, f2 = t2 == BOX || t2 == MESH;
  return (f1 && f2) || (t1 == CAPSULE && f2) || (f1 && t2 == CAPSULE);
}

bool encloses_origin(const Polytope& p) {
  if (p.nvert < 4 || p.nface < 4) return false;
  for (int i = 0; i < p.nface; ++i) {
    int f = p.face[i];
    V a = p.vertex(f & 1023), b = p.vertex((f >> 10) & 1023), c = p.vertex((f >> 20) & 1023);
    V u = b - a, v = c - a, n = crs(u, v);
    T origin = -dot(n, a), center = dot(n, p.center - a);
    if (center == 0 || (origin > 0 && center < 0) || (origin < 0 && center > 0)) return false;
  }
  return true;
}

Epa epa_phase(T tol, int iters, Gjk r, const CGeom& a, const CGeom& b, int t1, int t2, Polytope& p, bool require_enclosing) {
  p.nface = p.nvert = p.nhorizon = p.status = 0;
  if (r.dim == 2) polytope_segment(p, r, a, b, t1, t2);
  else if (r.dim == 4) polytope_tetrahedron(p, r);
  if (r.dim == 3) polytope_triangle(p, r, a, b, t1, t2, require_enclosing);
  if (p.status) return Epa{r.dist, 1, r.x1, r.x2, -1};
  if (require_enclosing && !encloses_origin(p)) return Epa{r.dist, 1, r.x1, r.x2, -1};
  bool discrete = discrete_pair(t1, t2) && a.margin == 0 && b.margin == 0;
  Epa e = epa_expand(tol, iters, p, a, b, t1, t2, discrete);
  if (!multicontact_supported(a, b, t1, t2)) e.face = -1;
  return e;
}

int simplex_to_face(const Gjk& r, Polytope& p) {
  for (int i = 0; i < 3; ++i) {
    int k = r.dim > i ? i : 0;
    p.vert[2 * i] = r.s1[k]; p.vert[2 * i + 1] = r.s2[k];
    p.vidx[2 * i] = r.v1[k]; p.vidx[2 * i + 1] = r.v2[k];
  }
  p.face[0] = (1 << 10) + (2 << 20);
  return 0;
}

// ------------------------------------------------------------------ box-box manifold
struct Manifold { int count; V one[4], two[4]; T distance[4]; };
struct Feature { int dim, index[3]; V point[3]; };
struct Normals { int count, index[3]; V normal[3]; };

Feature box_feature(const Polytope& p, int face, int side) {
  int ids[3] = {face & 1023, (face >> 10) & 1023, (face >> 20) & 1023};
  Feature f{};
  for (int i = 0; i < 3; ++i) { f.index[i] = p.vidx[2 * ids[i] + side]; f.point[i] = p.vert[2 * ids[i] + side]; }
  if (f.index[0] != f.index[1]) f.dim = (f.index[2] == f.index[0] || f.index[2] == f.index[1]) ? 2 : 3;
  else { f.index[1] = f.index[2]; f.point[1] = f.point[2]; f.dim = f.index[0] != f.index[2] ? 2 : 1; }
  return f;
}

V face_normal(int i) { V n = mk(0, 0, 0); n[i / 2] = (i % 2) == 0 ? 1 : -1; return n; }

const T kAlign = 0.99605101346969604, kPerp = 0.088782943785190582;

Normals normals_near(const CGeom& g, V d) {
  Normals n{};
  V local = unit(rotT(g.rot, d));
  for (int i = 0; i < 6; ++i)
    if (dot(local, face_normal(i)) > kAlign) { n.count = 1; n.normal[0] = rot(g.rot, face_normal(i)); n.index[0] = i; return n; }
  return n;
}

Normals box_normals(const CGeom& g, const Feature& f, V d) {
  Normals n{};
  if (f.dim == 3) {
    V common = mk(0, 0, 0);
    int count = 0;
    for (int k = 0; k < 3; ++k) {
      int bit = 1 << k;
      T value = T((f.index[0] & bit) && (f.index[1] & bit) && (f.index[2] & bit)) -
                T(!(f.index[0] & bit) && !(f.index[1] & bit) && !(f.index[2] & bit));
      common[k] = value;
      if (value != 0) n.index[count++] = 2 * k;
    }
    if (common[0] + common[1] + common[2] == -1) ++n.index[0];
    if (count == 1) { n.count = 1; n.normal[0] = rot(g.rot, common); return n; }
    return normals_near(g, d);
  }
  if (f.dim == 2) {
    for (int k = 0; k < 3; ++k) {
      int bit = 1 << k;
      T value = T((f.index[0] & bit) && (f.index[1] & bit)) - T(!(f.index[0] & bit) && !(f.index[1] & bit));
      if (value != 0) {
        int i = n.count++;
        V local = mk(0, 0, 0);
        local[k] = value;
        n.normal[i] = rot(g.rot, local);
        n.index[i] = 2 * k + (value > 0 ? 0 : 1);
      }
    }
    if (n.count == 1 || n.count == 2) return n;
    return normals_near(g, d);
  }
  if (f.dim == 1) {
    n.count = 3;
    for (int k = 0; k < 3; ++k) {
      int i = 2 * k + ((f.index[0] & (1 << k)) ? 0 : 1);
      n.index[k] = i;
      n.normal[k] = rot(g.rot, face_normal(i));
    }
  }
  return n;
}

Normals edge_normals(const CGeom& g, const Feature& f, V* end) {
  Normals n{};
  if (f.dim == 2) { end[0] = f.point[1]; n.normal[0] = unit(f.point[1] - f.point[0]); n.count = 1; }
  if (f.dim == 1) {
    V local;
    for (int k = 0; k < 3; ++k) local[k] = (f.index[0] & (1 << k)) ? g.size[k] : -g.size[k];
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

int box_face(const CGeom& g, int face, V* out) {
  const int corners[6][4] = {{7, 3, 1, 5}, {2, 6, 4, 0}, {2, 3, 7, 6}, {4, 5, 1, 0}, {6, 7, 5, 4}, {3, 2, 0, 1}};
  for (int i = 0; i < 4; ++i) {
    V pt;
    for (int k = 0; k < 3; ++k) pt[k] = (corners[face][i] & (1 << k)) ? g.size[k] : -g.size[k];
    out[i] = rot(g.rot, pt) + g.pos;
  }
  return 4;
}

T quad_area(V a, V b, V c, V d) { V n = crs(a - c, b - d); return 0.5 * std::sqrt(dot(n, n)); }

// Four polygon points of (locally) maximal quadrilateral area, by rotating calipers-like advances.
void polygon_quad(const V* p, int count, int* res) {
  int b = 1, c = 2, d = 3;
  res[0] = 0; res[1] = b; res[2] = c; res[3] = d;
  T area = quad_area(p[0], p[b], p[c], p[d]);
  for (int a = 0; a < count; ++a) {
    while (true) {
      T next = quad_area(p[a], p[b], p[c], p[(d + 1) % count]);
      if (next <= area) break;
      area = next; d = (d + 1) % count;
      res[0] = a; res[1] = b; res[2] = c; res[3] = d;
      while (true) {
        next = quad_area(p[a], p[b], p[(c + 1) % count], p[d]);
        if (next <= area) break;
        area = next; c = (c + 1) % count;
        res[0] = a; res[1] = b; res[2] = c; res[3] = d;
      }
      while (true) {
        next = quad_area(p[a], p[(b + 1) % count], p[c], p[d]);
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

// Clip polygon face2 against the side planes of face1 (normal `normal`), keep the points behind
// face1's plane, reduce to at most 4 (2 for an edge); witnesses are the clipped points (on geom 2's
// feature) and their projections back along `direction` (on geom 1's feature).
Manifold polygon_clip(const V* face1, int n1, const V* face2, int n2, V normal, V direction) {
  Manifold res{};
  if (n1 < 3) return res;
  V normals[4], buf1[8], buf2[8];
  T plane[4];
  V* poly = buf1;
  V* clipped = buf2;
  for (int i = 0; i < n1; ++i) {
    normals[i] = crs(face1[(i + 1) % n1] - face1[i], (face1[i] + normal) - face1[i]);
    plane[i] = dot(normals[i], face1[i]);
  }
  int count = n2;
  for (int i = 0; i < n2; ++i) poly[i] = face2[i];
  for (int e = 0; e < n1; ++e) {
    int nc = 0;
    for (int i = 0; i < count; ++i) {
      V p = poly[i], q = poly[(i + 1) % count];
      bool in1 = dot(p - face1[e], normals[e]) > -1e-10, in2 = dot(q - face1[e], normals[e]) > -1e-10;
      if (!in1 && !in2) continue;
      if (in1 && in2) { clipped[nc++] = q; continue; }
      T den = dot(normals[e], q - p);
      T t = std::fabs(den) < 1e-10 ? kFloatMax : (plane[e] - dot(normals[e], p)) / den;
      if (t > -3e-7 && t < 1 + 3e-7) { t = std::min(T(1), std::max(T(0), t)); clipped[nc++] = p + t * (q - p); }
      if (in2) clipped[nc++] = q;
    }
    std::swap(poly, clipped);
    count = nc;
  }
  int kept = 0;
  for (int i = 0; i < count; ++i) if (dot(poly[i] - face1[0], normal) <= 0) poly[kept++] = poly[i];
  count = kept;
  if (count < 1) return res;
  int ids[4] = {0, 1, 2, 3};
  if (n2 == 2 && count > 2) {
    T mx = 0;
    ids[0] = 0; ids[1] = 1;
    for (int i = 0; i < count; ++i)
      for (int j = i + 1; j < count; ++j) {
        V d = poly[j] - poly[i];
        T l = dot(d, d);
        if (l > mx) { mx = l; ids[0] = i; ids[1] = j; }
      }
    res.count = 2;
  } else if (count > 4) {
    polygon_quad(poly, count, ids);
    res.count = 4;
  } else {
    res.count = count;
  }
  for (int i = 0; i < res.count; ++i) {
    V v = poly[ids[i]];
    T d = dot(v - face1[0], normal);
    res.one[i] = v - direction * std::fabs(d);
    res.two[i] = v;
    res.distance[i] = d;
  }
  return res;
}

Manifold box_multicontact(const Polytope& p, int face, V x1, V x2, const CGeom& a, const CGeom& b) {
  Manifold fallback{};
  fallback.count = 1; fallback.one[0] = x1; fallback.two[0] = x2;
  Feature one = box_feature(p, p.face[face], 0), two = box_feature(p, p.face[face], 1);
  V dir = x2 - x1, end[3];
  Normals n1 = box_normals(a, one, -dir), n2 = box_normals(b, two, dir);
  int i = 0, j = 0, edge1 = 0, edge2 = 0;
  bool aligned = false;
  for (int k = 0; k < n1.count && !aligned; ++k)
    for (int l = 0; l < n2.count; ++l)
      if (dot(n1.normal[k], n2.normal[l]) < -kAlign) { i = k; j = l; aligned = true; break; }
  if (!aligned) {
    if (one.dim < 3 && n2.count && (one.dim <= two.dim || !n1.count)) {
      n1 = edge_normals(a, one, end);
      for (int k = 0; k < n2.count && !aligned; ++k) {
        if (dot(n2.normal[k], dir) <= kConvexMin) continue;
        for (int l = 0; l < n1.count; ++l)
          if (std::fabs(dot(n1.normal[l], n2.normal[k])) < kPerp) { i = l; j = k; aligned = true; break; }
      }
      if (!aligned) return fallback;
      edge1 = 1;
    } else if (two.dim < 3) {
      n2 = edge_normals(b, two, end);
      for (int k = 0; k < n1.count && !aligned; ++k) {
        if (dot(n1.normal[k], -dir) <= kConvexMin) continue;
        for (int l = 0; l < n2.count; ++l)
          if (std::fabs(dot(n2.normal[l], n1.normal[k])) < kPerp) { i = l; j = k; aligned = true; break; }
      }
      if (!aligned) return fallback;
      edge2 = 1;
    } else {
      return fallback;
    }
  }
  V face1[4], face2[4];
  int c1, c2;
  if (edge1) { face1[0] = one.point[0]; face1[1] = end[i]; c1 = 2; }
  else c1 = box_face(a, n1.index[edge2 ? j : i], face1);
  if (edge2) { face2[0] = two.point[0]; face2[1] = end[i]; c2 = 2; }
  else c2 = box_face(b, n2.index[j], face2);
  if (edge1) {
    Manifold r = polygon_clip(face2, c2, face1, c1, n2.normal[j], -n2.normal[j]);
    for (int k = 0; k < r.count; ++k) std::swap(r.one[k], r.two[k]);
    return r;
  }
  if (edge2) return polygon_clip(face1, c1, face2, c2, n1.normal[j], -n1.normal[j]);
  return polygon_clip(face1, c1, face2, c2, n1.normal[i], n2.normal[j]);
}

CGeom cgeom(const Geom& g, V pos, T margin) {
  CGeom c;
  c.pos = pos;
  c.size = mk(g.size[0], g.size[1], g.size[2]);
  c.rot = g.mat;
  c.vert = g.vert;
  c.nvert = g.type == MESH ? g.nvert : 0;
  c.cached = -1;
  c.margin = margin;
  return c;
}

}  // namespace

int g_horizon_capacity = 24;

// One convex pair in the translated frame of geom 1 (mjwarp_convex_collision.cuh:43-79).
int convex_pair(const Geom& g1, const Geom& g2, T margin, T gap, const CcdOptions& opt, std::vector<Raw>& out) {
  int t1 = g1.type, t2 = g2.type;
  V origin = ld(g1.pos);
  CGeom one = cgeom(g1, mk(0, 0, 0), margin), two = cgeom(g2, ld(g2.pos) - origin, margin);
  Phase ph = gjk_phase(opt.tolerance, gap, opt.iterations, one, two, t1, t2, one.pos, two.pos);
  Epa res{ph.distance, 1, ph.x1, ph.x2, -1};
  Polytope p(10 + 2 * opt.epa_iterations, 6 + 5 * opt.epa_iterations, g_horizon_capacity);
  if (ph.needs_epa) res = epa_phase(opt.tolerance, opt.epa_iterations, ph.r, ph.g1, ph.g2, t1, t2, p, ph.require_enclosing);
  // horizon overflow (mjwarp_convex_epa.cuh:186-214): no contact, the world is flagged
  if (res.horizon_overflow && opt.overflow) *opt.overflow |= MX_OVERFLOW_EPA_HORIZON;
  if (res.distance >= gap) return 1;
  T distance = res.distance + margin;
  Manifold mf{};
  mf.count = res.ncontact; mf.one[0] = res.x1; mf.two[0] = res.x2;
  if (t1 == BOX && t2 == BOX) {
    if (!ph.needs_epa && distance < 0 && margin == 0 && ph.r.dim > 0) res.face = simplex_to_face(ph.r, p);
    if (res.face >= 0) {
      mf = box_multicontact(p, res.face, res.x1, res.x2, ph.g1, ph.g2);
      if (mf.count < 1) { mf.count = 1; mf.one[0] = res.x1; mf.two[0] = res.x2; }
    }
  }
  V n = unit(distance <= margin ? mf.one[0] - mf.two[0] : mf.two[0] - mf.one[0]);
  T thr = margin + gap;
  for (int i = 0; i < mf.count; ++i) {
    T d = mf.count > 1 ? mf.distance[i] : distance;
    if (!(d < thr)) continue;
    V pos = 0.5 * (mf.one[i] + mf.two[i]) + origin;
    push(out, pos.v, n.v, d);
  }
  return 1;
}


// ------------------------------------------------------------------ MPR (MuJoCo 2.3.7)
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
// One convex pair by Minkowski Portal Refinement, MuJoCo 2.3.7's mjc_Convex with multiccd off:
// libccd's ccdMPRPenetration (portal discovery from the centre ray, refinement, penetration by
// portal expansion to mpr_tolerance; zero and equality tests against the route's epsilon),
// support points inflated by half the margin, the contact at the mean of the
// portal's support points on the two geoms, and the normal of a sphere or capsule side replaced by
// its surface normal (mjc_fixNormal).  Restated from libccd's published algorithm and MuJoCo's
// sources as vendored in gpu/host/runtime/collision/native_originals/ (ccd_mpr.c.txt,
// ccd_vec3.c.txt, engine_collision_convex.c.txt:42-240, 875-1017).  Portal discovery and refinement
// are bounded by mpr_iterations here (the originals loop until they decide).
namespace {
// The zero and equality threshold (CCD_EPS) of the route being restated: the reference's FP32 route
// builds libccd with ccd_real_t = float and CCD_EPS = FLT_EPSILON (gpu/cuda/common/precision.cuh:13-16,
// gpu/cuda/collision/native/native_source.cuh:555-559), its FP64 route and MuJoCo with DBL_EPSILON.
// The threshold decides branches (an absolute test on a squared cross product treats centre rays
// within about 2 degrees of a support point as collinear at FLT_EPSILON), so it is the route's,
// not the arithmetic's.  Set per pair by mpr_pair on the calling thread.
thread_local T kMprEps = 1.1920928955078125e-7;
bool mzero(T x) { return std::fabs(x) < kMprEps; }
bool meq(T a, T b) {
  T ab = std::fabs(a - b);
  if (ab < kMprEps) return true;
  return ab < kMprEps * std::max(std::fabs(a), std::fabs(b));
}
bool vorigin(V a) { return meq(a[0], 0) && meq(a[1], 0) && meq(a[2], 0); }
V vnorm(V a) { return a * (1 / std::sqrt(dot(a, a))); }
struct MSup { V v, v1, v2; };
struct MprGeoms { const CGeom* a; const CGeom* b; int ta, tb; };
// MuJoCo's support point (mjccd_support): a box coordinate takes sign(d) * size with sign(0) = 0, a
// hull the first vertex of largest projection; every shape inflated by half the margin
V mj_support(const CGeom& g, int type, V d) {
  if (type == SPHERE) return g.pos + (g.size[0] + 0.5 * g.margin) * d;
  V local = rotT(g.rot, d), res = mk(0, 0, 0);
  if (type == BOX) {
    for (int k = 0; k < 3; ++k) res[k] = sgn(local[k]) * g.size[k];
  } else if (type == CAPSULE) {
    res = local * g.size[0];
    res[2] += sgn(local[2]) * g.size[1];
  } else if (type == MESH) {
    T best = -1e10;
    for (int i = 0; i < g.nvert; ++i) {
      V v = ld(g.vert + 3 * i);
      T h = dot(v, local);
      if (h > best) { best = h; res = v; }
    }
  }
  res = res + local * (0.5 * g.margin);
  return rot(g.rot, res) + g.pos;
}
MSup msup(const MprGeoms& g, V d) {
  MSup s;
  s.v1 = mj_support(*g.a, g.ta, d);
  s.v2 = mj_support(*g.b, g.tb, -d);
  s.v = s.v1 - s.v2;
  return s;
}
V portal_dir(const MSup* p) { return vnorm(crs(p[2].v - p[1].v, p[3].v - p[1].v)); }
bool reach_tolerance(const MSup* p, const MSup& v4, V dir, T tol) {
  T d4 = dot(v4.v, dir);
  T m = std::min(d4 - dot(p[1].v, dir), std::min(d4 - dot(p[2].v, dir), d4 - dot(p[3].v, dir)));
  return meq(m, tol) || m < tol;
}
void expand(MSup* p, const MSup& v4) {
  V c = crs(v4.v, p[0].v);
  if (dot(p[1].v, c) > 0) {
    if (dot(p[2].v, c) > 0) p[1] = v4; else p[3] = v4;
  } else {
    if (dot(p[3].v, c) > 0) p[2] = v4; else p[1] = v4;
  }
}
// squared distance of the origin from segment (x0, b), with its witness
T seg_dist2(V x0, V b, V& w) {
  V d = b - x0, a = x0;
  T t = -dot(a, d) / dot(d, d);
  if (t < 0 || mzero(t)) w = x0;
  else if (t > 1 || meq(t, 1)) w = b;
  else w = x0 + t * d;
  return dot(w, w);
}
// squared distance of the origin from triangle (x0, b, c), with its witness
T tri_dist2(V x0, V b, V c, V& w) {
  V d1 = b - x0, d2 = c - x0, a = x0;
  T v = dot(d1, d1), ww = dot(d2, d2), p = dot(a, d1), q = dot(a, d2), r = dot(d1, d2);
  T d = ww * v - r * r, s, t;
  if (mzero(d)) { s = t = -1; }
  else { s = (q * r - ww * p) / d; t = (-s * r - q) / ww; }
  if ((mzero(s) || s > 0) && (meq(s, 1) || s < 1) && (mzero(t) || t > 0) && (meq(t, 1) || t < 1) &&
      (meq(t + s, 1) || t + s < 1)) {
    w = x0 + s * d1 + t * d2;
    return dot(w, w);
  }
  V w2;
  T dist = seg_dist2(x0, b, w);
  T d2b = seg_dist2(x0, c, w2);
  if (d2b < dist) { dist = d2b; w = w2; }
  d2b = seg_dist2(b, c, w2);
  if (d2b < dist) { dist = d2b; w = w2; }
  return dist;
}
// -1 no contact; 0 portal built; 1 origin at v1 (touching); 2 origin on segment v0-v1
int discover_portal(const MprGeoms& g, MSup* p, int maxit) {
  p[0].v1 = g.a->pos; p[0].v2 = g.b->pos; p[0].v = p[0].v1 - p[0].v2;
  if (vorigin(p[0].v)) p[0].v[0] += kMprEps * 10;
  V dir = vnorm(-p[0].v);
  p[1] = msup(g, dir);
  T dt = dot(p[1].v, dir);
  if (mzero(dt) || dt < 0) return -1;
  dir = crs(p[0].v, p[1].v);
  if (mzero(dot(dir, dir))) return vorigin(p[1].v) ? 1 : 2;
  dir = vnorm(dir);
  p[2] = msup(g, dir);
  dt = dot(p[2].v, dir);
  if (mzero(dt) || dt < 0) return -1;
  dir = vnorm(crs(p[1].v - p[0].v, p[2].v - p[0].v));
  if (dot(dir, p[0].v) > 0) { std::swap(p[1], p[2]); dir = -dir; }
  for (int it = 0; it < maxit; ++it) {
    p[3] = msup(g, dir);
    dt = dot(p[3].v, dir);
    if (mzero(dt) || dt < 0) return -1;
    bool cont = false;
    dt = dot(crs(p[1].v, p[3].v), p[0].v);
    if (dt < 0 && !mzero(dt)) { p[2] = p[3]; cont = true; }
    if (!cont) {
      dt = dot(crs(p[3].v, p[2].v), p[0].v);
      if (dt < 0 && !mzero(dt)) { p[1] = p[3]; cont = true; }
    }
    if (!cont) return 0;
    dir = vnorm(crs(p[1].v - p[0].v, p[2].v - p[0].v));
  }
  return -1;
}
V portal_pos(const MSup* p) {
  V dir = portal_dir(p);
  T b[4];
  b[0] = dot(crs(p[1].v, p[2].v), p[3].v);
  b[1] = dot(crs(p[3].v, p[2].v), p[0].v);
  b[2] = dot(crs(p[0].v, p[1].v), p[3].v);
  b[3] = dot(crs(p[2].v, p[1].v), p[0].v);
  T sum = b[0] + b[1] + b[2] + b[3];
  if (mzero(sum) || sum < 0) {
    b[0] = 0;
    b[1] = dot(crs(p[2].v, p[3].v), dir);
    b[2] = dot(crs(p[3].v, p[1].v), dir);
    b[3] = dot(crs(p[1].v, p[2].v), dir);
    sum = b[1] + b[2] + b[3];
  }
  T inv = 1 / sum;
  V p1 = mk(0, 0, 0), p2 = mk(0, 0, 0);
  for (int i = 0; i < 4; ++i) { p1 = p1 + b[i] * p[i].v1; p2 = p2 + b[i] * p[i].v2; }
  return 0.5 * (p1 * inv + p2 * inv);
}
// libccd ccdMPRPenetration: 0 with depth, dir, pos, or -1 (no penetration)
int mpr_penetration(const MprGeoms& g, T tol, int maxit, T& depth, V& dir, V& pos) {
  MSup p[4];
  int res = discover_portal(g, p, maxit);
  if (res < 0) return -1;
  if (res == 1) {   // touching at v1: no direction
    depth = 0; dir = mk(0, 0, 0); pos = 0.5 * (p[1].v1 + p[1].v2);
    return 0;
  }
  if (res == 2) {   // origin on segment v0-v1
    pos = 0.5 * (p[1].v1 + p[1].v2);
    dir = p[1].v;
    depth = std::sqrt(dot(dir, dir));
    dir = vnorm(dir);
    return 0;
  }
  for (int it = 0;; ++it) {   // refine the portal until it encloses the origin
    if (it >= maxit) return -1;
    V d = portal_dir(p);
    T e = dot(d, p[1].v);
    if (mzero(e) || e > 0) break;
    MSup v4 = msup(g, d);
    T c4 = dot(v4.v, d);
    if (!(mzero(c4) || c4 > 0) || reach_tolerance(p, v4, d, tol)) return -1;
    expand(p, v4);
  }
  for (int it = 0;; ++it) {   // expand towards the boundary for the penetration
    V d = portal_dir(p);
    MSup v4 = msup(g, d);
    if (reach_tolerance(p, v4, d, tol) || it > maxit) {
      V w;
      depth = std::sqrt(tri_dist2(p[1].v, p[2].v, p[3].v, w));
      dir = mzero(depth) ? mk(0, 0, 0) : vnorm(w);
      pos = portal_pos(p);
      return 0;
    }
    expand(p, v4);
  }
}
// mjc_fixNormal: a sphere's or capsule's surface normal at the contact point replaces the MPR
// normal (both: their difference, normalized)
V fix_normal(const Geom& g1, const Geom& g2, V pos_world, V frame) {
  V normal[2] = {frame, -frame};
  bool done[2] = {false, false};
  const Geom* gg[2] = {&g1, &g2};
  for (int i = 0; i < 2; ++i) {
    int t = gg[i]->type;
    if (t != SPHERE && t != CAPSULE) continue;
    V local = rotT(gg[i]->mat, pos_world - ld(gg[i]->pos)), nrm;
    if (t == SPHERE) {
      nrm = local;
    } else {
      T h = gg[i]->size[1];
      nrm = mk(local[0], local[1], local[2] < -h ? local[2] + h : (local[2] > h ? local[2] - h : 0));
    }
    T n = std::sqrt(dot(nrm, nrm));
    nrm = n < 1e-15 ? mk(1, 0, 0) : nrm * (1 / n);
    normal[i] = rot(gg[i]->mat, nrm);
    done[i] = true;
  }
  if (done[0] && done[1]) {
    V d = normal[0] - normal[1];
    T n = std::sqrt(dot(d, d));
    return n < 1e-15 ? mk(1, 0, 0) : d * (1 / n);
  }
  if (done[0]) return normal[0];
  if (done[1]) return -normal[1];
  return frame;
}
}  // namespace

int mpr_pair(const Geom& g1, const Geom& g2, T margin, T gap, T tolerance, int iterations, T eps,
             std::vector<Raw>& out) {
  // mjc_Convex (engine_collision_convex.c.txt:278-296): each shape inflated by margin / 2, one
  // contact at margin - depth; the gap does not widen detection (it lowers includemargin only)
  (void)gap;
  const T thr = margin;
  kMprEps = eps;
  // geom 1's centre as the frame origin (a common translation leaves the portal's geometry)
  V origin = ld(g1.pos);
  CGeom a = cgeom(g1, ld(g1.pos) - origin, thr), b = cgeom(g2, ld(g2.pos) - origin, thr);
  MprGeoms g{&a, &b, g1.type, g2.type};
  T depth;
  V dir, pos;
  if (mpr_penetration(g, tolerance, iterations, depth, dir, pos) != 0) return 1;
  if (vorigin(dir)) return 1;   // contact without a normal: none
  V pw = pos + origin;
  V n = fix_normal(g1, g2, pw, dir);
  push(out, pw.v, n.v, thr - depth);
  return 1;
}

}  // namespace narrow
}  // namespace orc
