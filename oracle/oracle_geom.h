// Geometry shared by the oracle's narrowphase files -- TEST INFRASTRUCTURE ONLY (see oracle.h).
#pragma once
#include "oracle_internal.h"

namespace orc {
inline namespace narrow {

enum { PLANE = 0, SPHERE = 2, CAPSULE = 3, BOX = 6, MESH = 7 };

// Hull polygons of a mesh geom: per polygon (mesh-local ids) the first entry in `vert` (an
// absolute index), the count and the outward normal (geom frame); per vertex of the mesh the first
// entry in `map` (absolute) and the count of the polygons that contain it.
struct MeshPolys {
  int npoly = 0;
  const int *vertadr = nullptr, *vertnum = nullptr, *vert = nullptr;
  const T* normal = nullptr;
  const int *mapadr = nullptr, *mapnum = nullptr, *map = nullptr;
};

struct Geom {
  int id, type;
  T pos[3], mat[9], size[3];
  const T* vert = nullptr;
  int nvert = 0;
  MeshPolys poly;
};

struct Raw {   // one contact before material assignment
  T pos[3], normal[3], dist;
  bool has_tangent = false;   // plane-capsule fixes the second frame axis itself
  T tangent[3] = {0, 0, 0};
};

inline void axis(const T* mat, int k, T* out) { out[0] = mat[k]; out[1] = mat[3 + k]; out[2] = mat[6 + k]; }

inline void normalize3(T* v) {
  T n = norm3(v);
  if (n > kMinVal) { v[0] /= n; v[1] /= n; v[2] /= n; }
}

// MJWarp make_frame: tangent from y (or z when the normal is close to y), then the cross product.
inline void make_frame(const T* n, T* frame) {
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

inline void push(std::vector<Raw>& out, const T* pos, const T* normal, T dist) {
  Raw r;
  for (int k = 0; k < 3; ++k) { r.pos[k] = pos[k]; r.normal[k] = normal[k]; }
  r.dist = dist;
  out.push_back(r);
}

// Convex pairs (GJK / EPA, box-box manifold); returns 1 when the pair family is handled.
// `overflow` (may be null) collects MX_OVERFLOW_EPA_HORIZON when a polytope's horizon edge list
// exceeds its capacity (the pair then gives no contact, as the reference's epa_horizon_overflow).
struct CcdOptions {
  T tolerance;
  int iterations, epa_iterations;
  int* overflow;
  int mpr = 0;             // convex pairs by MPR (MuJoCo 2.3.7) instead of GJK/EPA
  T mpr_tolerance = 1e-6;
  int mpr_iterations = 50;
  // MPR's zero and equality threshold: FLT_EPSILON for the reference's FP32 route (the device
  // kernel's), DBL_EPSILON for its FP64 route and MuJoCo's double build
  T mpr_eps = 1.1920928955078125e-7;
};
// Horizon edge capacity of the EPA polytope (24, the device kernel's kHorizon); tests shrink it.
extern int g_horizon_capacity;
int convex_pair(const Geom& g1, const Geom& g2, T margin, T gap, const CcdOptions& opt, std::vector<Raw>& out);
// One convex pair by MPR (MuJoCo 2.3.7 mjc_Convex, one contact): detection threshold margin + gap,
// zero and equality tests against eps.
int mpr_pair(const Geom& g1, const Geom& g2, T margin, T gap, T tolerance, int iterations, T eps,
             std::vector<Raw>& out);

}  // namespace narrow
}  // namespace orc
