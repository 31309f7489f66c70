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
#include "oracle_geom.h"

namespace orc {
inline namespace narrow {

// ------------------------------------------------------------------ plane
// Plane routines restate gpu/cuda/collision/mjwarp_plane.cu:18-39; `thr` = margin + gap.
void plane_point(const Geom& p, const T* c, T r, T thr, std::vector<Raw>& out) {
  T n[3];
  axis(p.mat, 2, n);
  T d[3] = {c[0] - p.pos[0], c[1] - p.pos[1], c[2] - p.pos[2]};
  T dist = dot3(n, d) - r;
  if (!(dist < thr)) return;
  T pos[3];
  for (int k = 0; k < 3; ++k) pos[k] = c[k] - n[k] * (r + 0.5 * dist);
  push(out, pos, n, dist);
}

// both end spheres, the +axis end first; the frame's second axis is the capsule axis projected on
// the plane (mjwarp_plane.cu:22-31)
void plane_capsule(const Geom& p, const Geom& cap, T thr, std::vector<Raw>& out) {
  T n[3], ax[3];
  axis(p.mat, 2, n);
  axis(cap.mat, 2, ax);
  T proj = dot3(n, ax);
  T b[3] = {ax[0] - n[0] * proj, ax[1] - n[1] * proj, ax[2] - n[2] * proj};
  T len = norm3(b);
  if (len != 0) for (int k = 0; k < 3; ++k) b[k] /= len;
  if (len < 0.5) {
    b[0] = 0;
    b[1] = (-0.5 < n[1] && n[1] < 0.5) ? 1 : 0;
    b[2] = (-0.5 < n[1] && n[1] < 0.5) ? 0 : 1;
  }
  for (int e = 1; e >= -1; e -= 2) {
    T c[3];
    for (int k = 0; k < 3; ++k) c[k] = cap.pos[k] + e * ax[k] * cap.size[1];
    size_t before = out.size();
    plane_point(p, c, cap.size[0], thr, out);
    if (out.size() > before) {
      out.back().has_tangent = true;
      for (int k = 0; k < 3; ++k) out.back().tangent[k] = b[k];
    }
  }
}

// every box corner within the threshold, in corner order (mjwarp_plane.cu:32-39)
void plane_box(const Geom& p, const Geom& box, T thr, std::vector<Raw>& out) {
  T n[3];
  axis(p.mat, 2, n);
  T dc[3] = {box.pos[0] - p.pos[0], box.pos[1] - p.pos[1], box.pos[2] - p.pos[2]};
  T center_dist = dot3(dc, n);
  for (int i = 0; i < 8; ++i) {
    T l[3] = {(i & 1) ? box.size[0] : -box.size[0], (i & 2) ? box.size[1] : -box.size[1],
              (i & 4) ? box.size[2] : -box.size[2]};
    T corner[3];
    mulmv3(box.mat, l, corner);
    T dist = center_dist + dot3(n, corner);
    if (!(dist < thr)) continue;
    T pos[3];
    for (int k = 0; k < 3; ++k) pos[k] = corner[k] + box.pos[k] - 0.5 * n[k] * dist;
    push(out, pos, n, dist);
  }
}

// Area of the quadrilateral (polygon vertices i, j, k, l): half the norm of the diagonals' cross
// product (quadrilateral_area, gpu/cuda/collision/mjwarp_plane.cu:53-57).
T quad_area(const Geom& g, int face, int i, int j, int k, int l) {
  const int* pv = g.poly.vert + face;
  const T *a = g.vert + 3 * pv[i], *b = g.vert + 3 * pv[j], *c = g.vert + 3 * pv[k], *d = g.vert + 3 * pv[l];
  T u[3] = {a[0] - c[0], a[1] - c[1], a[2] - c[2]}, v[3] = {b[0] - d[0], b[1] - d[1], b[2] - d[2]}, x[3];
  cross(u, v, x);
  return 0.5 * norm3(x);
}

// Up to four polygon corners spanning the largest quadrilateral, grown from the anchor corner by
// advancing the last, then the third, then the second corner while the area grows (hull4,
// mjwarp_plane.cu:58-79).
int hull4(const Geom& g, int face, int count, int anchor, int* idx) {
  int b = (anchor + 1) % count, c = (anchor + 2) % count, d = (anchor + 3) % count;
  idx[0] = anchor; idx[1] = b; idx[2] = c; idx[3] = d;
  if (count <= 4) return count;
  T area = quad_area(g, face, anchor, b, c, d);
  while (true) {
    int next = (d + 1) % count;
    T cand = quad_area(g, face, anchor, b, c, next);
    if (cand <= area) break;
    d = next; area = cand; idx[1] = b; idx[2] = c; idx[3] = d;
    while (true) {
      next = (c + 1) % count;
      cand = quad_area(g, face, anchor, b, next, d);
      if (cand <= area) break;
      c = next; area = cand; idx[1] = b; idx[2] = c; idx[3] = d;
    }
    while (true) {
      next = (b + 1) % count;
      cand = quad_area(g, face, anchor, next, c, d);
      if (cand <= area) break;
      b = next; area = cand; idx[1] = b; idx[2] = c; idx[3] = d;
    }
  }
  return 4;
}

// Convex mesh against a plane (plane_mesh, mjwarp_plane.cu:80-121): the support vertex along the
// plane's inward normal; when it lies within the threshold, the corners of the incident polygon
// whose normal is most opposed to the plane normal (hull4 of them), those below the geom centre.
// Candidates at or beyond `thr` are dropped as the reference's publish step drops them.
void plane_mesh(const Geom& p, const Geom& g, T thr, std::vector<Raw>& out) {
  T n[3], ln[3];
  axis(p.mat, 2, n);
  for (int k = 0; k < 3; ++k) ln[k] = g.mat[k] * n[0] + g.mat[3 + k] * n[1] + g.mat[6 + k] * n[2];
  int index = -1;
  T best = -1e10;
  for (int i = 0; i < g.nvert; ++i) {
    T s = -dot3(ln, g.vert + 3 * i);
    if (s > best) { best = s; index = i; }
  }
  if (index < 0) return;
  auto world = [&](int i, T* w) {
    mulmv3(g.mat, g.vert + 3 * i, w);
    for (int k = 0; k < 3; ++k) w[k] += g.pos[k];
  };
  auto emit = [&](const T* v) {
    T d[3] = {v[0] - p.pos[0], v[1] - p.pos[1], v[2] - p.pos[2]}, dist = dot3(n, d), pos[3];
    for (int k = 0; k < 3; ++k) pos[k] = v[k] - 0.5 * dist * n[k];
    if (dist < thr) push(out, pos, n, dist);
    return dist;
  };
  T v0[3];
  world(index, v0);
  T dist = emit(v0);
  if (g.poly.npoly <= 0 || dist > thr) return;
  int best_poly = -1;
  T best_dot = 1;
  for (int i = 0; i < g.poly.mapnum[index]; ++i) {
    int id = g.poly.map[g.poly.mapadr[index] + i];
    T dt = dot3(g.poly.normal + 3 * id, ln);
    if (dt < best_dot) { best_dot = dt; best_poly = id; }
  }
  if (best_poly < 0) return;
  int face = g.poly.vertadr[best_poly], count = g.poly.vertnum[best_poly], anchor = 0;
  for (int i = 0; i < count; ++i)
    if (g.poly.vert[face + i] == index) { anchor = i; break; }
  int idx[4];
  int hull = hull4(g, face, count, anchor, idx);
  for (int i = 1; i < hull; ++i) {
    T v[3];
    world(g.poly.vert[face + idx[i]], v);
    T d[3] = {v[0] - g.pos[0], v[1] - g.pos[1], v[2] - g.pos[2]};
    if (dot3(n, d) > 0) continue;
    emit(v);
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

// ------------------------------------------------------------------ sphere / capsule / box
// Restatement of MJWarp's primitive box routines as the reference ships them
// (gpu/cuda/collision/mjwarp_box.cu), in double.  `thr` is the detection threshold margin + gap.
constexpr T kBoxMin = 1e-15, kBoxMax = 1e10;

T clampd(T v, T lo, T hi) { return std::max(lo, std::min(hi, v)); }
T safe_div(T x, T y) { return x / (y != 0 ? y : kBoxMin); }

// sphere (centre c, radius r) as geom 1 against box geom 2 (mjwarp_box.cu:14-32)
void sphere_box(const T* c, T r, const Geom& box, T thr, std::vector<Raw>& out) {
  T d[3] = {c[0] - box.pos[0], c[1] - box.pos[1], c[2] - box.pos[2]}, local[3], clamped[3];
  mulmtv3(box.mat, d, local);
  for (int k = 0; k < 3; ++k) clamped[k] = clampd(local[k], -box.size[k], box.size[k]);
  T dir[3] = {clamped[0] - local[0], clamped[1] - local[1], clamped[2] - local[2]};
  T len = norm3(dir);
  if (len != 0) for (int k = 0; k < 3; ++k) dir[k] /= len;
  T lpos[3], lnormal[3], dist;
  if (len <= kBoxMin) {
    // centre inside: push out through the nearest face
    T closest = 2 * (box.size[0] + box.size[1] + box.size[2]);
    int face = 0;
    for (int i = 0; i < 6; ++i) {
      T f = std::fabs(((i % 2) ? 1 : -1) * box.size[i / 2] - local[i / 2]);
      if (closest > f) { closest = f; face = i; }
    }
    T nearest[3] = {0, 0, 0};
    nearest[face / 2] = (face % 2) ? -1 : 1;
    for (int k = 0; k < 3; ++k) { lpos[k] = local[k] + nearest[k] * (r - closest) * 0.5; lnormal[k] = nearest[k]; }
    dist = -closest - r;
  } else {
    for (int k = 0; k < 3; ++k) {
      T deepest = local[k] + dir[k] * r;
      lpos[k] = 0.5 * (clamped[k] + deepest);
      lnormal[k] = dir[k];
    }
    dist = len - r;
  }
  if (!(dist < thr)) return;
  T wpos[3], n[3];
  mulmv3(box.mat, lpos, wpos);
  mulmv3(box.mat, lnormal, n);
  for (int k = 0; k < 3; ++k) wpos[k] += box.pos[k];
  push(out, wpos, n, dist);
}

// capsule geom 1 against box geom 2 (mjwarp_box.cu:33-102): the closest feature pair of segment and
// box (end caps, then the 12 box edges in corner-major order), a sphere contact there and, when
// the segment lies along a face, a second sphere contact further along the segment.
void capsule_box(const Geom& cap, const Geom& box, T thr, std::vector<Raw>& out) {
  T radius = cap.size[0], half = cap.size[1];
  T d[3] = {cap.pos[0] - box.pos[0], cap.pos[1] - box.pos[1], cap.pos[2] - box.pos[2]}, pos[3], wax[3], ax[3];
  mulmtv3(box.mat, d, pos);
  axis(cap.mat, 2, wax);
  mulmtv3(box.mat, wax, ax);
  const T* size = box.size;
  T ha[3] = {ax[0] * half, ax[1] * half, ax[2] * half};
  int axisdir = int(ha[0] > 0) + 2 * int(ha[1] > 0) + 4 * int(ha[2] > 0);
  T bestdist = 1e32, bestsegment = -12, bestbox = 0;
  int type = -4, face = -12, corner = -123, edge = -123;
  for (int i = -1; i <= 1; i += 2) {
    T tip[3], pt[3];
    int outside = 0, a = -1;
    for (int k = 0; k < 3; ++k) { tip[k] = pos[k] + i * ha[k]; pt[k] = tip[k]; }
    for (int j = 0; j < 3; ++j) {
      if (pt[j] < -size[j]) { ++outside; a = j; pt[j] = -size[j]; }
      else if (pt[j] > size[j]) { ++outside; a = j; pt[j] = size[j]; }
    }
    if (outside > 1) continue;
    T dif[3] = {pt[0] - tip[0], pt[1] - tip[1], pt[2] - tip[2]};
    T dd = dot3(dif, dif);
    if (dd < bestdist) { bestdist = dd; bestsegment = i; type = -2 + i; face = a; }
  }
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 3; ++j) {
      if (i & (1 << j)) continue;
      T pt[3] = {(i & 1) ? size[0] : -size[0], (i & 2) ? size[1] : -size[1], (i & 4) ? size[2] : -size[2]};
      pt[j] = 0;
      T dif[3] = {pt[0] - pos[0], pt[1] - pos[1], pt[2] - pos[2]};
      T u = -size[j] * dif[j], v = dot3(ha, dif), ma = size[j] * size[j], mb = -size[j] * ha[j], mc = half * half;
      T det = ma * mc - mb * mb;
      if (std::fabs(det) < kBoxMin) continue;
      T inv = 1 / det, x1 = (mc * u - mb * v) * inv, x2 = (ma * v - mb * u) * inv;
      int s1 = 1, s2 = 1;
      if (x1 > 1) { x1 = 1; s1 = 2; x2 = safe_div(v - mb, mc); }
      else if (x1 < -1) { x1 = -1; s1 = 0; x2 = safe_div(v + mb, mc); }
      bool over = x2 > 1;
      if (over || x2 < -1) {
        if (over) { x2 = 1; s2 = 2; x1 = safe_div(u - mb, ma); }
        else { x2 = -1; s2 = 0; x1 = safe_div(u + mb, ma); }
        if (x1 > 1) { x1 = 1; s1 = 2; }
        else if (x1 < -1) { x1 = -1; s1 = 0; }
      }
      for (int k = 0; k < 3; ++k) dif[k] -= ha[k] * x2;
      dif[j] += size[j] * x1;
      T dd = dot3(dif, dif);
      int config = s1 * 3 + s2;
      if (dd < bestdist - kBoxMin) {
        bestdist = dd; bestsegment = x2; bestbox = x1;
        corner = i + (1 << j) * (config / 6); edge = j; type = config;
      }
    }
  if (type == -4) return;
  T second = -4;
  if (type >= 0 && type / 3 != 1) {
    int config = axisdir ^ corner;
    if (config != 0 && config != 7) {
      int mul;
      if (config == 1 || config == 2 || config == 4) mul = 1;
      else { mul = -1; config = 7 - config; }
      int a = config == 1 ? 0 : config == 2 ? 1 : 2, a1 = (a + 1) % 3, a2 = (a + 2) % 3;
      if (ax[a] * ax[a] > 0.5) {
        T mm = 2 * safe_div(size[a], std::fabs(ha[a]));
        second = std::min(1 - mul * bestsegment, mm);
      } else {
        T mm = 2 * std::min(safe_div(size[a1], std::fabs(ha[a1])), safe_div(size[a2], std::fabs(ha[a2])));
        second = -std::min(1 + mul * bestsegment, mm);
      }
      second *= mul;
    }
  } else if (type >= 0 && type / 3 == 1) {
    int config = (axisdir ^ corner) & (7 - (1 << edge));
    if (config == 1 || config == 2 || config == 4) {
      int a = edge, a1 = (edge + 1) % 3, a2 = (edge + 2) % 3;
      if (std::fabs(ax[a1]) > std::fabs(ax[a2])) a1 = a2;
      a2 = 3 - a - a1;
      int mul;
      if (config & (1 << a2)) { mul = 1; second = 1 - bestsegment; }
      else { mul = -1; second = 1 + bestsegment; }
      T e1 = 2 * safe_div(size[a2], std::fabs(ha[a2]));
      second = std::min(e1, second);
      T e2 = (bool(axisdir & (1 << a)) == bool(config & (1 << a2))) ? 1 - bestbox : 1 + bestbox;
      e1 = size[a] * safe_div(e2, std::fabs(ha[a]));
      second = std::min(e1, second);
      second *= mul;
    }
  } else if (type < 0 && face != -1) {
    int mul = type == -3 ? 1 : -1;
    second = 2;
    T tmp[3] = {pos[0] - ha[0] * mul, pos[1] - ha[1] * mul, pos[2] - ha[2] * mul};
    for (int i = 0; i < 3; ++i) {
      if (i == face) continue;
      T inv = safe_div(T(mul), ha[i]);
      T e1 = (size[i] - tmp[i]) * inv;
      if (0 < e1 && e1 < second) second = e1;
      e1 = (-size[i] - tmp[i]) * inv;
      if (0 < e1 && e1 < second) second = e1;
    }
    second *= mul;
  }
  auto sphere_at = [&](T t) {
    T l[3] = {pos[0] + ha[0] * t, pos[1] + ha[1] * t, pos[2] + ha[2] * t}, w[3];
    mulmv3(box.mat, l, w);
    for (int k = 0; k < 3; ++k) w[k] += box.pos[k];
    sphere_box(w, radius, box, thr, out);
  };
  sphere_at(bestsegment);
  if (second > -3) sphere_at(second + bestsegment);
}

// ------------------------------------------------------------------ box-box
// Clip the polygon (face-plane coordinates) against sign * p[coord] <= limit (mjwarp_box.cu:103-114).
int clip_face(int count, T (*poly)[3], int coord, T sign, T limit) {
  T d[8];
  bool inside = true;
  for (int i = 0; i < count; ++i) { d[i] = sign * poly[i][coord] - limit; if (!(d[i] <= 0)) inside = false; }
  if (inside) return count;
  T clipped[8][3] = {};
  int n = 0;
  for (int i = 0; i < count; ++i) {
    int next = i + 1 == count ? 0 : i + 1;
    T dp = d[i], dq = d[next];
    if (dp <= 0 && n < 8) { for (int k = 0; k < 3; ++k) clipped[n][k] = poly[i][k]; ++n; }
    if (((dp < 0 && dq > 0) || (dp > 0 && dq < 0)) && n < 8) {
      T t = dp / (dp - dq);
      for (int k = 0; k < 3; ++k) clipped[n][k] = poly[i][k] + t * (poly[next][k] - poly[i][k]);
      ++n;
    }
  }
  for (int i = 0; i < 8; ++i) for (int k = 0; k < 3; ++k) poly[i][k] = clipped[i][k];
  return n;
}

// Separating-axis test over the 3 + 3 face axes and 9 edge axes, then either one edge-edge contact
// or the incident face clipped against the reference face (mjwarp_box.cu:115-176).
void box_box(const Geom& g1, const Geom& g2, T margin, std::vector<Raw>& out) {
  const T *s1 = g1.size, *s2 = g2.size;
  T d21[3] = {g2.pos[0] - g1.pos[0], g2.pos[1] - g1.pos[1], g2.pos[2] - g1.pos[2]};
  T d12[3] = {-d21[0], -d21[1], -d21[2]}, pos21[3], pos12[3];
  mulmtv3(g1.mat, d21, pos21);
  mulmtv3(g2.mat, d12, pos12);
  T rot[9], ab[9];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      T a[3], b[3];
      axis(g1.mat, i, a);
      axis(g2.mat, j, b);
      rot[3 * i + j] = dot3(a, b);
      ab[3 * i + j] = std::fabs(rot[3 * i + j]);
    }
  T septol = margin + 1e-6 * (s1[0] + s1[1] + s1[2] + s2[0] + s2[1] + s2[2]), best = -kBoxMax;
  int code = -1;
  for (int i = 0; i < 3; ++i) {
    T radius = ab[3 * i] * s2[0] + ab[3 * i + 1] * s2[1] + ab[3 * i + 2] * s2[2];
    T sep = std::fabs(pos21[i]) - s1[i] - radius;
    if (sep > septol) return;
    if (sep > best) { best = sep; code = i; }
  }
  for (int j = 0; j < 3; ++j) {
    T radius = ab[j] * s1[0] + ab[3 + j] * s1[1] + ab[6 + j] * s1[2];
    T sep = std::fabs(pos12[j]) - s2[j] - radius;
    if (sep > septol) return;
    if (sep > best) { best = sep; code = 3 + j; }
  }
  T face_best = best;
  int face_code = code;
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      int i1 = (i + 1) % 3, i2 = (i + 2) % 3;
      T x = -rot[3 * i2 + j], y = rot[3 * i1 + j], n2 = x * x + y * y;
      if (n2 < 1e-7) continue;
      T inv = 1 / std::sqrt(n2);
      x *= inv; y *= inv;
      T r1 = s1[i1] * std::fabs(x) + s1[i2] * std::fabs(y);
      int j1 = (j + 1) % 3, j2 = (j + 2) % 3;
      T a1 = x * rot[3 * i1 + j1] + y * rot[3 * i2 + j1], a2 = x * rot[3 * i1 + j2] + y * rot[3 * i2 + j2];
      T r2 = s2[j1] * std::fabs(a1) + s2[j2] * std::fabs(a2);
      T sep = std::fabs(x * pos21[i1] + y * pos21[i2]) - r1 - r2;
      if (sep > septol) return;
      if (sep - 1e-6 * std::fabs(sep) > best && sep > face_best) { best = sep; code = 6 + 3 * i + j; }
    }
  if (code < 0) return;
  int ei = 0, ej = 0, i1 = 0, i2 = 0;
  T ax[3] = {0, 0, 0};
  if (code >= 6) {
    ei = (code - 6) / 3; ej = (code - 6) % 3; i1 = (ei + 1) % 3; i2 = (ei + 2) % 3;
    ax[i1] = -rot[3 * i2 + ej];
    ax[i2] = rot[3 * i1 + ej];
    normalize3(ax);
    T align;
    if (face_code < 3) align = std::fabs(ax[face_code]);
    else {
      T col[3] = {rot[face_code - 3], rot[3 + face_code - 3], rot[6 + face_code - 3]};
      align = std::fabs(dot3(ax, col));
    }
    if (align > 0.99 && best < face_best + 0.05 * std::fabs(face_best) + kBoxMin) { code = face_code; best = face_best; }
  }
  if (code >= 6) {
    int j1 = (ej + 1) % 3, j2 = (ej + 2) % 3;
    if (dot3(ax, pos21) < 0) for (int k = 0; k < 3; ++k) ax[k] = -ax[k];
    T a2[3];
    mulmtv3(rot, ax, a2);
    int amb1 = -1, amb2 = -1;
    if (std::fabs(ax[i1]) < 1e-5) amb1 = i1;
    else if (std::fabs(ax[i2]) < 1e-5) amb1 = i2;
    if (std::fabs(a2[j1]) < 1e-5) amb2 = j1;
    else if (std::fabs(a2[j2]) < 1e-5) amb2 = j2;
    T dv2[3] = {rot[ej], rot[3 + ej], rot[6 + ej]};
    T b = dv2[ei], denom = 1 - b * b, best_dist = kBoxMax;
    T w1[3] = {0, 0, 0}, w2[3] = {0, 0, 0};
    for (int v1 = 0; v1 < (amb1 >= 0 ? 2 : 1); ++v1)
      for (int v2 = 0; v2 < (amb2 >= 0 ? 2 : 1); ++v2) {
        T c1[3] = {0, 0, 0}, corner[3] = {0, 0, 0}, c2[3];
        c1[i1] = ax[i1] >= 0 ? s1[i1] : -s1[i1];
        c1[i2] = ax[i2] >= 0 ? s1[i2] : -s1[i2];
        if (amb1 >= 0 && v1) c1[amb1] = -c1[amb1];
        corner[j1] = a2[j1] >= 0 ? -s2[j1] : s2[j1];
        corner[j2] = a2[j2] >= 0 ? -s2[j2] : s2[j2];
        if (amb2 >= 0 && v2) corner[amb2] = -corner[amb2];
        mulmv3(rot, corner, c2);
        for (int k = 0; k < 3; ++k) c2[k] += pos21[k];
        T e[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
        T d1e = e[ei], d2e = dot3(dv2, e);
        T s = denom >= kBoxMin ? (d1e - b * d2e) / denom : 0;
        s = clampd(s, -s1[ei], s1[ei]);
        T t = clampd(b * s - d2e, -s2[ej], s2[ej]);
        s = clampd(d1e + b * t, -s1[ei], s1[ei]);
        T q1[3] = {c1[0], c1[1], c1[2]}, q2[3];
        q1[ei] = s;
        for (int k = 0; k < 3; ++k) q2[k] = c2[k] + dv2[k] * t;
        T g[3] = {q2[0] - q1[0], q2[1] - q1[1], q2[2] - q1[2]};
        T dd = dot3(g, g);
        if (dd < best_dist) { best_dist = dd; for (int k = 0; k < 3; ++k) { w1[k] = q1[k]; w2[k] = q2[k]; } }
      }
    T gap[3] = {w2[0] - w1[0], w2[1] - w1[1], w2[2] - w1[2]};
    T dist = dot3(gap, ax);
    if (dist > septol) return;
    T mid[3] = {0.5 * (w1[0] + w2[0]), 0.5 * (w1[1] + w2[1]), 0.5 * (w1[2] + w2[2])}, wpos[3], n[3];
    mulmv3(g1.mat, mid, wpos);
    for (int k = 0; k < 3; ++k) wpos[k] += g1.pos[k];
    mulmv3(g1.mat, ax, n);
    if (dist < margin) push(out, wpos, n, dist);
    return;
  }
  bool ref1 = code < 3;
  int a = ref1 ? code : code - 3;
  const T *size_ref = ref1 ? s1 : s2, *size_inc = ref1 ? s2 : s1, *pos_ref = ref1 ? g1.pos : g2.pos;
  const T* posoi = ref1 ? pos21 : pos12;
  const T* matref = ref1 ? g1.mat : g2.mat;
  T rinc[9];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) rinc[3 * i + j] = ref1 ? rot[3 * i + j] : rot[3 * j + i];
  T sign = posoi[a] >= 0 ? 1 : -1;
  int inc = 0;
  for (int k = 1; k < 3; ++k) if (std::fabs(rinc[3 * a + k]) > std::fabs(rinc[3 * a + inc])) inc = k;
  T incsign = sign * rinc[3 * a + inc] > 0 ? -1 : 1;
  int fx = (a + 1) % 3, fy = (a + 2) % 3, bu = (inc + 1) % 3, bv = (inc + 2) % 3, coords[3] = {fx, fy, a};
  T cx[3], du[3], dv[3];
  for (int r = 0; r < 3; ++r) {
    int c = coords[r];
    cx[r] = posoi[c] + incsign * size_inc[inc] * rinc[3 * c + inc];
    du[r] = size_inc[bu] * rinc[3 * c + bu];
    dv[r] = size_inc[bv] * rinc[3 * c + bv];
  }
  cx[2] = sign * cx[2] - size_ref[a];
  du[2] *= sign;
  dv[2] *= sign;
  T poly[8][3] = {};
  for (int k = 0; k < 4; ++k) {
    T su = (k == 0 || k == 3) ? 1 : -1, sv = k < 2 ? 1 : -1;
    for (int r = 0; r < 3; ++r) poly[k][r] = cx[r] + su * du[r] + sv * dv[r];
  }
  int count = 4;
  count = clip_face(count, poly, 0, 1, size_ref[fx]);
  count = clip_face(count, poly, 0, -1, size_ref[fx]);
  count = clip_face(count, poly, 1, 1, size_ref[fy]);
  count = clip_face(count, poly, 1, -1, size_ref[fy]);
  T kept[8][3];
  int accepted = 0;
  T duplicate = 1e-10 * (size_ref[fx] * size_ref[fx] + size_ref[fy] * size_ref[fy]);
  for (int k = 0; k < count; ++k) {
    if (poly[k][2] > margin) continue;
    bool dupe = false;
    for (int q = 0; q < accepted; ++q) {
      T dx = kept[q][0] - poly[k][0], dy = kept[q][1] - poly[k][1];
      if (dx * dx + dy * dy < duplicate) { dupe = true; break; }
    }
    if (!dupe) { for (int r = 0; r < 3; ++r) kept[accepted][r] = poly[k][r]; ++accepted; }
  }
  T n[3];
  axis(matref, a, n);
  T ns = ref1 ? sign : -sign;
  for (int k = 0; k < 3; ++k) n[k] *= ns;
  for (int k = 0; k < accepted; ++k) {
    T local[3] = {0, 0, 0}, wpos[3];
    local[fx] = kept[k][0];
    local[fy] = kept[k][1];
    local[a] = sign * (size_ref[a] + 0.5 * kept[k][2]);
    mulmv3(matref, local, wpos);
    for (int r = 0; r < 3; ++r) wpos[r] += pos_ref[r];
    if (kept[k][2] < margin) push(out, wpos, n, kept[k][2]);
  }
}

// ------------------------------------------------------------------ dispatch
// Pair dispatch: primitive routines take the detection threshold, margin + gap on the MJWarp route
// and the margin alone under MuJoCo 2.3.7 semantics (ccd.mpr: mj_collideGeoms calls the collision
// functions with the margin; the gap only lowers includemargin); convex pairs (hulls, and box-box
// unless the model selects the primitive SAT) go through GJK/EPA, or MPR under ccd.mpr.
int narrowphase(const Geom& g1, const Geom& g2, T mrg, T gap, const CcdOptions& ccd, bool boxbox_primitive,
                std::vector<Raw>& out) {
  int t1 = g1.type, t2 = g2.type;
  T margin = ccd.mpr ? mrg : mrg + gap;
  if (t1 != PLANE && (t2 == MESH || (t1 == BOX && t2 == BOX && !boxbox_primitive)))
    return ccd.mpr ? mpr_pair(g1, g2, mrg, gap, ccd.mpr_tolerance, ccd.mpr_iterations, ccd.mpr_eps, out)
                   : convex_pair(g1, g2, mrg, gap, ccd, out);
  if (t1 == PLANE) {
    if (t2 == SPHERE) plane_point(g1, g2.pos, g2.size[0], margin, out);
    else if (t2 == CAPSULE) plane_capsule(g1, g2, margin, out);
    else if (t2 == BOX) plane_box(g1, g2, margin, out);
    else if (t2 == MESH) plane_mesh(g1, g2, margin, out);
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
  return 0;
}

}  // namespace

void collision(const OrModel& m, World& w, const int32_t* body_active) {
  w.contacts.clear();
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
      int padr = m.mesh_polyadr[id];
      x.poly.npoly = m.mesh_polynum[id];
      x.poly.vertadr = m.mesh_polyvertadr + padr;
      x.poly.vertnum = m.mesh_polyvertnum + padr;
      x.poly.vert = m.mesh_polyvert;
      x.poly.normal = m.mesh_polynormal + 3 * padr;
      x.poly.mapadr = m.mesh_polymapadr + m.mesh_vertadr[id];
      x.poly.mapnum = m.mesh_polymapnum + m.mesh_vertadr[id];
      x.poly.map = m.mesh_polymap;
    }
    return x;
  };
  for (int p = 0; p < m.npair; ++p) {
    int g1 = m.pair_geom[2 * p], g2 = m.pair_geom[2 * p + 1];
    if (body_active && (!body_active[m.geom_body[g1]] || !body_active[m.geom_body[g2]])) continue;
    // MJWarp route: margins and gaps add (contact_material, mjwarp_contact.cuh:71-72) and a contact
    // is detected below margin + gap; MuJoCo 2.3.7 (convex_mpr; the reference's native route,
    // collision/collision_dispatch.cuh:115-116, as mj_collideGeoms): the larger margin and the
    // larger gap, detected below the margin.  The constraint row uses margin - gap either way.
    T margin, gap, thr;
    if (m.convex_mpr) {
      margin = std::max(m.geom_margin[g1], m.geom_margin[g2]);
      gap = std::max(m.geom_gap[g1], m.geom_gap[g2]);
      thr = margin;
    } else {
      margin = m.geom_margin[g1] + m.geom_margin[g2];
      gap = m.geom_gap[g1] + m.geom_gap[g2];
      thr = margin + gap;
    }
    // broadphase: plane half-space or bounding spheres (mjwarp_broadphase.cu:20-27)
    const T* c1 = &w.geom_xpos[3 * g1];
    const T* c2 = &w.geom_xpos[3 * g2];
    if (m.geom_type[g1] == PLANE) {
      T n[3] = {w.geom_xmat[9 * g1 + 2], w.geom_xmat[9 * g1 + 5], w.geom_xmat[9 * g1 + 8]};
      T d[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
      if (dot3(n, d) > m.geom_rbound[g2] + thr) continue;
    } else {
      T d[3] = {c2[0] - c1[0], c2[1] - c1[1], c2[2] - c1[2]};
      T bound = m.geom_rbound[g1] + m.geom_rbound[g2] + thr;
      if (dot3(d, d) > bound * bound) continue;
    }
    std::vector<Raw> raw;
    CcdOptions ccd{m.opt_ccd_tolerance, m.opt_ccd_iterations, m.epa_iterations, &w.overflow, m.convex_mpr,
                   m.opt_mpr_tolerance, m.opt_mpr_iterations};
    narrowphase(geom(g1), geom(g2), margin, gap, ccd, m.boxbox_primitive != 0, raw);
    // material (contact_material, mjwarp_contact.cuh:56-101): the priority winner's condim and
    // friction, else the larger of each; solref / solimp mixed by solmix (weight 1 or 0 for a
    // priority winner), solref by element-wise minimum when either uses the direct format
    int pr1 = m.geom_priority[g1], pr2 = m.geom_priority[g2];
    int dim;
    T fr[3], solref[2], solimp[5], mix;
    if (pr1 != pr2) {
      int g = pr1 > pr2 ? g1 : g2;
      mix = pr1 > pr2 ? 1 : 0;
      dim = m.geom_condim[g];
      for (int k = 0; k < 3; ++k) fr[k] = m.geom_friction[3 * g + k];
    } else {
      dim = std::max(m.geom_condim[g1], m.geom_condim[g2]);
      for (int k = 0; k < 3; ++k) fr[k] = std::max(m.geom_friction[3 * g1 + k], m.geom_friction[3 * g2 + k]);
      T s1 = m.geom_solmix[g1], s2 = m.geom_solmix[g2];
      mix = s1 + s2 != 0 ? s1 / (s1 + s2) : 0;
      if (s1 < kMinVal && s2 < kMinVal) mix = 0.5;
      if (s1 < kMinVal && s2 >= kMinVal) mix = 0;
      if (s1 >= kMinVal && s2 < kMinVal) mix = 1;
    }
    if (m.geom_solref[2 * g1] > 0 && m.geom_solref[2 * g2] > 0)
      for (int k = 0; k < 2; ++k) solref[k] = mix * m.geom_solref[2 * g1 + k] + (1 - mix) * m.geom_solref[2 * g2 + k];
    else
      for (int k = 0; k < 2; ++k) solref[k] = std::min(m.geom_solref[2 * g1 + k], m.geom_solref[2 * g2 + k]);
    for (int k = 0; k < 5; ++k) solimp[k] = mix * m.geom_solimp[5 * g1 + k] + (1 - mix) * m.geom_solimp[5 * g2 + k];
    for (int k = 0; k < 3; ++k) fr[k] = std::max(T(1e-5), fr[k]);
    for (const Raw& r : raw) {
      if ((int)w.contacts.size() >= m.nconmax) { w.overflow |= MX_OVERFLOW_NARROWPHASE; break; }
      Contact c;
      for (int k = 0; k < 3; ++k) c.pos[k] = r.pos[k];
      make_frame(r.normal, c.frame);
      if (r.has_tangent) {
        for (int k = 0; k < 3; ++k) { c.frame[k] = r.normal[k]; c.frame[3 + k] = r.tangent[k]; }
        cross(r.normal, r.tangent, c.frame + 6);
      }
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

namespace {
// Polygon pack of one mesh for or_collide: ints = {npoly, nvert, vertadr[npoly], vertnum[npoly],
// mapadr[nvert], mapnum[nvert], polygon vertex lists..., vertex polygon lists...} (offsets local to
// the lists), normals = 3 per polygon.
void unpack_polys(orc::Geom& g, const int* ints, const double* normals) {
  if (!ints) return;
  int np = ints[0], nv = ints[1];
  g.poly.npoly = np;
  g.poly.vertadr = ints + 2;
  g.poly.vertnum = ints + 2 + np;
  g.poly.mapadr = ints + 2 + 2 * np;
  g.poly.mapnum = ints + 2 + 2 * np + nv;
  g.poly.vert = ints + 2 + 2 * np + 2 * nv;
  int total = 0;
  for (int i = 0; i < np; ++i) total += g.poly.vertnum[i];
  g.poly.map = g.poly.vert + total;
  g.poly.normal = normals;
}
thread_local int g_last_collide_flags = 0;
}  // namespace

// Test hooks: the overflow bits of the last or_collide call on this thread, and the EPA horizon
// capacity (24 as on the device; tests shrink it to force an overflow).
extern "C" int or_last_collide_flags(void) { return g_last_collide_flags; }
// The contact frame the step publishes for a contact normal (make_frame; rows: normal, tangent,
// normal x tangent), for the frame-convention pins.
extern "C" void or_contact_frame(const double* normal, double* frame) { orc::make_frame(normal, frame); }
extern "C" void or_set_horizon_capacity(int capacity) { orc::narrow::g_horizon_capacity = capacity > 0 ? capacity : 24; }

extern "C" int or_collide(int type1, const double* pos1, const double* mat1, const double* size1,
                          const double* vert1, int nvert1, const int* poly1, const double* pnorm1,
                          int type2, const double* pos2, const double* mat2,
                          const double* size2, const double* vert2, int nvert2, const int* poly2,
                          const double* pnorm2, double margin, double gap,
                          int boxbox_primitive, double ccd_tolerance, int ccd_iterations, int epa_iterations,
                          double* out_pos, double* out_normal, double* out_dist, int maxout) {
  using namespace orc;
  Geom g1, g2;
  g1.id = 0; g1.type = type1; g2.id = 1; g2.type = type2;
  for (int k = 0; k < 3; ++k) { g1.pos[k] = pos1[k]; g1.size[k] = size1[k]; g2.pos[k] = pos2[k]; g2.size[k] = size2[k]; }
  for (int k = 0; k < 9; ++k) { g1.mat[k] = mat1[k]; g2.mat[k] = mat2[k]; }
  g1.vert = vert1; g1.nvert = nvert1; g2.vert = vert2; g2.nvert = nvert2;
  unpack_polys(g1, poly1, pnorm1);
  unpack_polys(g2, poly2, pnorm2);
  std::vector<Raw> raw;
  int flags = 0;
  // boxbox_primitive: bit 0 primitive box-box, bit 1 convex pairs by MPR (tolerance and iterations
  // then the MPR ones), bit 2 MPR's tests against DBL_EPSILON (MuJoCo's double build) instead of
  // FLT_EPSILON (the reference's FP32 route)
  CcdOptions ccd{ccd_tolerance, ccd_iterations, epa_iterations, &flags, (boxbox_primitive >> 1) & 1,
                 ccd_tolerance, ccd_iterations};
  if ((boxbox_primitive >> 2) & 1) ccd.mpr_eps = 2.220446049250313e-16;
  if (!narrowphase(g1, g2, margin, gap, ccd, (boxbox_primitive & 1) != 0, raw)) return -1;
  g_last_collide_flags = flags;
  int n = std::min((int)raw.size(), maxout);
  for (int i = 0; i < n; ++i) {
    for (int k = 0; k < 3; ++k) { out_pos[3 * i + k] = raw[i].pos[k]; out_normal[3 * i + k] = raw[i].normal[k]; }
    out_dist[i] = raw[i].dist;
  }
  return n;
}
