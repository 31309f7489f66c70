// Constraint rows and the Newton solver of the CPU FP64 oracle -- TEST INFRASTRUCTURE ONLY.
//
// Rows restate gpu/cuda/dynamics/mjwarp_constraint_build.cu (impedance :22-37, publish_row :39-48,
// dof friction :62, joint limits :77, contact allocation :95, contact Jacobian :124 with pyramidal
// and elliptic rows :137-145, reference rows :161-199), in a deterministic order (friction rows by
// dof, limit rows by joint, contact rows by contact and component) instead of per-world atomics.
// The solver restates MJWarp's dense Newton as the reference runs it:
//   initialize_world        gpu/cuda/newton/mjwarp_solver_state.cu:61-92
//   constraint_gradient     gpu/cuda/newton/mjwarp_constraint.cu:107-201
//   mass_quadratic / cone   gpu/cuda/newton/mjwarp_hessian.cu:33-212
//   direction + stopping    gpu/cuda/newton/mjwarp_direction.cu:120-158
//   iterative_search        gpu/cuda/newton/mjwarp_linesearch.cu:81-375
#include "oracle_internal.h"

namespace orc {
namespace {

enum { kSatisfied = 0, kQuadratic = 1, kLinearNeg = 2, kLinearPos = 3, kCone = 4 };
enum { EFC_FRICTION = 1, EFC_LIMIT = 3, EFC_FRICTIONLESS = 5, EFC_PYRAMIDAL = 6, EFC_ELLIPTIC = 7 };

struct KBI { T k, b, imp; };

// solref/solimp -> stiffness k, damping b, impedance at `position` (mjwarp_constraint_build.cu:22-37)
KBI impedance(T timestep, const T* ref, const T* imp, T position) {
  const T minimp = 0.0001, maximp = 0.9999;
  auto clamp = [](T x, T lo, T hi) { return std::min(std::max(x, lo), hi); };
  T time = std::max(ref[0], 2 * timestep);   // refsafe
  T lo = clamp(imp[0], minimp, maximp), hi = clamp(imp[1], minimp, maximp);
  T width = std::max(kMinVal, imp[2]), mid = clamp(imp[3], minimp, maximp), power = std::max(T(1), imp[4]);
  T k = ref[0] <= 0 ? -ref[0] / std::max(kMinVal, hi * hi) : 1 / std::max(kMinVal, hi * hi * time * time * ref[1] * ref[1]);
  T b = ref[1] <= 0 ? -ref[1] / std::max(kMinVal, hi) : 2 / std::max(kMinVal, hi * time);
  T x = std::fabs(position) / width, r;
  if (lo == hi || imp[2] <= kMinVal) r = 0.5 * (lo + hi);
  else if (x <= 0) r = lo;
  else if (x >= 1) r = hi;
  else if (power == 1) r = lo + x * (hi - lo);
  else if (x <= mid) r = clamp(lo + (1 / std::pow(mid, power - 1)) * std::pow(x, power) * (hi - lo), lo, hi);
  else r = clamp(lo + (1 - (1 / std::pow(1 - mid, power - 1)) * std::pow(1 - x, power)) * (hi - lo), lo, hi);
  return {k, b, r};
}

void publish_row(const OrModel& m, World& w, int r, T position, T impedance_position, T weight,
                 const T* ref, const T* imp, T margin, T velocity, T friction, int type, int id) {
  KBI kbi = impedance(m.opt_timestep, ref, imp, impedance_position);
  T k = type == EFC_FRICTION ? 0 : kbi.k;
  w.D[r] = 1 / std::max(weight * (1 - kbi.imp) / kbi.imp, kMinVal);
  w.aref[r] = -k * kbi.imp * position - kbi.b * velocity;
  w.efc_vel[r] = velocity;
  w.efc_pos[r] = position + margin;
  w.frictionloss[r] = friction;
  w.type[r] = type;
  w.id[r] = id;
}

void resize_rows(const OrModel& m, World& w, int n) {
  w.J.assign((size_t)n * m.nv, 0);
  for (auto* v : {&w.D, &w.aref, &w.efc_pos, &w.efc_vel, &w.frictionloss, &w.force, &w.jaref, &w.jv}) v->assign(n, 0);
  w.quad.assign(3 * (size_t)n, 0);
  w.type.assign(n, 0);
  w.id.assign(n, 0);
  w.state.assign(n, 0);
}

}  // namespace

// Translational/rotational Jacobian of a point attached to `body` (MuJoCo mj_jac).
void body_jac(const OrModel& m, const World& w, int body, const T* point, T* jacp, T* jacr) {
  int r = m.body_rootid[body];
  T off[3];
  for (int k = 0; k < 3; ++k) off[k] = point[k] - w.subtree_com[3 * r + k];
  std::fill(jacp, jacp + 3 * m.nv, 0.0);
  std::fill(jacr, jacr + 3 * m.nv, 0.0);
  if (body == 0) return;
  for (int d = m.body_lastdof[body]; d >= 0; d = m.dof_parent[d]) {
    const T* c = &w.cdof[6 * d];
    T t[3];
    cross(c, off, t);
    for (int k = 0; k < 3; ++k) {
      jacr[k * m.nv + d] = c[k];
      jacp[k * m.nv + d] = c[3 + k] + t[k];
    }
  }
}

void make_constraint(const OrModel& m, World& w, const T* qpos, const T* qvel) {
  int nv = m.nv;
  w.ne = w.nf = w.nl = w.nefc = 0;
  if (m.opt_disableflags & 1) { resize_rows(m, w, 0); return; }
  // count rows first (deterministic order: friction, limits, contacts)
  std::vector<int> frows, lrows;
  if (!(m.opt_disableflags & (1 << 2)))
    for (int d = 0; d < nv; ++d) if (m.dof_frictionloss[d] > 0) frows.push_back(d);
  std::vector<T> lpos;
  std::vector<T> lsign;
  if (!(m.opt_disableflags & (1 << 3)))
    for (int j = 0; j < m.njnt; ++j) {
      int type = m.jnt_type[j];
      if (!m.jnt_limited[j] || (type != 2 && type != 3)) continue;
      T q = qpos[m.jnt_qposadr[j]];
      T lower = q - m.jnt_range[2 * j], upper = m.jnt_range[2 * j + 1] - q;
      T position = std::min(lower, upper) - m.jnt_margin[j];
      if (!(position < 0)) continue;
      lrows.push_back(j);
      lpos.push_back(position);
      lsign.push_back(lower < upper ? 1.0 : -1.0);
    }
  std::vector<int> crow_count(w.contacts.size(), 0);
  int ncrows = 0;
  for (size_t c = 0; c < w.contacts.size(); ++c) {
    const Contact& ct = w.contacts[c];
    T position = ct.dist - ct.includemargin;
    if (!(position < 0)) continue;
    int dim = ct.dim;
    crow_count[c] = (m.opt_cone == 1 || dim == 1) ? dim : 2 * (dim - 1);
    ncrows += crow_count[c];
  }
  int total = (int)frows.size() + (int)lrows.size() + ncrows;
  int cap = std::min(total, m.njmax);
  if (total > m.njmax) w.overflow |= MX_OVERFLOW_NEFC;
  resize_rows(m, w, cap);
  int r = 0;
  // dof friction rows (mjwarp_constraint_build.cu:62-75)
  for (int d : frows) {
    if (r >= cap) break;
    w.J[(size_t)r * nv + d] = 1;
    publish_row(m, w, r, 0, 0, m.dof_invweight0[d], m.dof_solref + 2 * d, m.dof_solimp + 5 * d, 0, qvel[d],
                m.dof_frictionloss[d], EFC_FRICTION, d);
    ++r; ++w.nf;
  }
  // joint limit rows (mjwarp_constraint_build.cu:77-93)
  for (size_t k = 0; k < lrows.size(); ++k) {
    if (r >= cap) break;
    int j = lrows[k], d = m.jnt_dofadr[j];
    w.J[(size_t)r * nv + d] = lsign[k];
    publish_row(m, w, r, lpos[k], lpos[k], m.dof_invweight0[d], m.jnt_solref + 2 * j, m.jnt_solimp + 5 * j,
                m.jnt_margin[j], lsign[k] * qvel[d], 0, EFC_LIMIT, j);
    ++r; ++w.nl;
  }
  // contact rows (mjwarp_constraint_build.cu:95-199)
  std::vector<T> jp1(3 * nv), jr1(3 * nv), jp2(3 * nv), jr2(3 * nv);
  T ratio = 1 / std::sqrt(m.opt_impratio);
  for (size_t c = 0; c < w.contacts.size(); ++c) {
    Contact& ct = w.contacts[c];
    ct.efc_address = -1;
    int count = crow_count[c];
    if (!count) continue;
    if (r + count > cap) { r = cap; break; }
    ct.efc_address = r;
    int b1 = m.geom_body[ct.geom[0]], b2 = m.geom_body[ct.geom[1]];
    body_jac(m, w, b1, ct.pos, jp1.data(), jr1.data());
    body_jac(m, w, b2, ct.pos, jp2.data(), jr2.data());
    int dim = ct.dim;
    const T* fr = ct.friction;
    T weight = m.body_invweight0[2 * b1] + m.body_invweight0[2 * b2];
    T position = ct.dist - ct.includemargin;
    for (int comp = 0; comp < count; ++comp, ++r) {
      T* J = &w.J[(size_t)r * nv];
      for (int d = 0; d < nv; ++d) {
        T lin[3], ang[3];
        for (int k = 0; k < 3; ++k) {
          lin[k] = jp2[k * nv + d] - jp1[k * nv + d];
          ang[k] = jr2[k * nv + d] - jr1[k * nv + d];
        }
        T v;
        if (m.opt_cone == 1) {
          v = dot3(comp < 3 ? lin : ang, ct.frame + 3 * (comp % 3));
        } else {
          v = dot3(lin, ct.frame);
          if (dim > 1) {
            int dir = comp / 2 + 1;
            T f = fr[dir - 1] * (1 - 2 * T(comp & 1));
            v += dot3(dir < 3 ? lin : ang, ct.frame + 3 * (dir % 3)) * f;
          }
        }
        J[d] = v;
      }
      T vel = 0;
      for (int d = 0; d < nv; ++d) vel += J[d] * qvel[d];
      T wgt = weight, pos_aref = position, scale = 1;
      if (m.opt_cone == 1 && comp > 0) {
        scale = ratio * ratio;
        if (comp > 1) scale *= fr[0] * fr[0] / (fr[comp - 1] * fr[comp - 1]);
        pos_aref = 0;
      } else if (m.opt_cone == 0 && dim > 1) {
        wgt = wgt + fr[0] * fr[0] * wgt;
        wgt = wgt * 2 * fr[0] * fr[0] * ratio * ratio;
      }
      int type = dim == 1 ? EFC_FRICTIONLESS : (m.opt_cone == 1 ? EFC_ELLIPTIC : EFC_PYRAMIDAL);
      publish_row(m, w, r, pos_aref, position, wgt, ct.solref, ct.solimp, ct.includemargin, vel, 0, type, (int)c);
      if (m.opt_cone == 1 && comp > 0) {
        w.D[r] /= scale;
        w.aref[r] = -impedance(m.opt_timestep, ct.solref, ct.solimp, position).b * vel;
      }
    }
  }
  w.nefc = r;
}

namespace {

// ------------------------------------------------------------------ Newton pieces
T safe_div(T x, T y) { return x / (y != 0 ? y : 1e-15); }

struct Point {
  T cost, slope, curv;
  Point operator+(const Point& b) const { return {cost + b.cost, slope + b.slope, curv + b.curv}; }
};

// elliptic cone data of a contact from current Jaref (constraint_gradient, mjwarp_constraint.cu:124-170)
struct ConeRow { int head; T mu, n, t, tt, d0; };

// row forces and states, qfrc_constraint = J^T f, grad = Ma - qfrc_smooth - J^T f
void gradient(const OrModel& m, World& w) {
  int nv = m.nv, R = w.nefc;
  T ratio = 1 / std::sqrt(m.opt_impratio);
  for (int r = 0; r < R; ++r) {
    T d = w.D[r], res = w.jaref[r];
    bool equality = r < w.ne, friction = !equality && r < w.ne + w.nf;
    T force;
    int state;
    if (equality) { force = -d * res; state = kQuadratic; }
    else if (friction) {
      T loss = w.frictionloss[r], rad = safe_div(loss, d);
      if (res <= -rad) { force = loss; state = kLinearNeg; }
      else if (res >= rad) { force = -loss; state = kLinearPos; }
      else { force = -d * res; state = kQuadratic; }
    } else if (w.type[r] == EFC_ELLIPTIC) {
      const Contact& ct = w.contacts[w.id[r]];
      int head = ct.efc_address;
      T mu = ct.friction[0] * ratio;
      T normal = w.jaref[head], d0 = w.D[head], tt = 0, tscale = 0;
      for (int j = 1; j < ct.dim; ++j) {
        T u = w.jaref[head + j] * ct.friction[j - 1];
        tt += u * u;
        if (r == head + j) tscale = u * ct.friction[j - 1];
      }
      T n = normal * mu, t = tt <= 0 ? 0 : std::sqrt(tt);
      if (n >= mu * t || (t <= 0 && n >= 0)) { force = 0; state = kSatisfied; }
      else if (mu * n + t <= 0 || (t <= 0 && n < 0)) { force = -d * res; state = kQuadratic; }
      else {
        T dm = safe_div(d0, mu * mu * (1 + mu * mu));
        T fn = -dm * (n - mu * t) * mu;
        force = r == head ? fn : -safe_div(fn, t) * tscale;
        state = kCone;
      }
    } else if (res >= 0) { force = 0; state = kSatisfied; }
    else { force = -d * res; state = kQuadratic; }
    w.force[r] = force;
    w.state[r] = state;
  }
  for (int i = 0; i < nv; ++i) {
    T s = 0;
    for (int r = 0; r < R; ++r) s += w.J[(size_t)r * nv + i] * w.force[r];
    w.qfrc_constraint[i] = s;
    w.grad[i] = w.Ma[i] - w.qfrc_smooth[i] - s;
  }
}

// H = M + sum over quadratic rows of D J^T J, plus elliptic cone curvature (mjwarp_hessian.cu)
void hessian(const OrModel& m, World& w) {
  int nv = m.nv, R = w.nefc;
  std::fill(w.H.begin(), w.H.end(), 0.0);
  for (int t = 0; t < m.ntree; ++t) {
    int n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < n; ++j) w.H[(size_t)(a + i) * nv + a + j] = w.M[m.tree_madr[t] + i * n + j];
  }
  for (int r = 0; r < R; ++r) {
    if (w.state[r] != kQuadratic) continue;
    const T* J = &w.J[(size_t)r * nv];
    T d = w.D[r];
    for (int i = 0; i < nv; ++i) {
      if (J[i] == 0) continue;
      for (int j = 0; j < nv; ++j) w.H[(size_t)i * nv + j] += d * J[i] * J[j];
    }
  }
  if (m.opt_cone != 1) return;
  T ratio = 1 / std::sqrt(m.opt_impratio);
  for (const Contact& ct : w.contacts) {
    int head = ct.efc_address;
    if (head < 0 || ct.dim == 1 || w.state[head] != kCone) continue;
    T mu = ct.friction[0] * ratio, mu2 = mu * mu;
    T den = mu2 * (1 + mu2);
    T dm = w.D[head] / (den != 0 ? den : kMinVal);
    if (dm == 0) continue;
    T n = w.jaref[head] * mu;
    T tt = 0;
    for (int d = 1; d < ct.dim; ++d) { T u = w.jaref[head + d] * ct.friction[d - 1]; tt += u * u; }
    T t = std::max(std::sqrt(tt), kMinVal), it = 1 / t, mnt = mu * n * it;
    for (int i = 0; i < nv; ++i)
      for (int j = 0; j < nv; ++j) {
        T z01 = mu * w.J[(size_t)head * nv + i], z02 = mu * w.J[(size_t)head * nv + j];
        T p1 = 0, p2 = 0, td = 0;
        for (int d = 1; d < ct.dim; ++d) {
          T sc = ct.friction[d - 1], u = w.jaref[head + d] * sc;
          T z1 = sc * w.J[(size_t)(head + d) * nv + i], z2 = sc * w.J[(size_t)(head + d) * nv + j];
          p1 += u * z1; p2 += u * z2; td += z1 * z2;
        }
        p1 *= it; p2 *= it;
        w.H[(size_t)i * nv + j] += dm * (z01 * z02 - mu * (z01 * p2 + z02 * p1) + mnt * p1 * p2 + (mu2 - mnt) * td);
      }
  }
}

// search = -H^-1 grad (dense Cholesky), search_dot, decrement
void direction(const OrModel& m, World& w, T& search_dot, T& decrement) {
  int n = m.nv;
  std::vector<T>& F = w.Hf;
  F = w.H;
  for (int j = 0; j < n; ++j) {
    T d = F[(size_t)j * n + j];
    for (int k = 0; k < j; ++k) d -= F[(size_t)j * n + k] * F[(size_t)j * n + k];
    d = std::sqrt(std::max(d, kMinVal));
    F[(size_t)j * n + j] = d;
    for (int i = j + 1; i < n; ++i) {
      T v = F[(size_t)i * n + j];
      for (int k = 0; k < j; ++k) v -= F[(size_t)i * n + k] * F[(size_t)j * n + k];
      F[(size_t)i * n + j] = v / d;
    }
  }
  std::vector<T> x(w.grad.begin(), w.grad.end());
  for (int i = 0; i < n; ++i) {
    T s = x[i];
    for (int k = 0; k < i; ++k) s -= F[(size_t)i * n + k] * x[k];
    x[i] = s / F[(size_t)i * n + i];
  }
  for (int i = n - 1; i >= 0; --i) {
    T s = x[i];
    for (int k = i + 1; k < n; ++k) s -= F[(size_t)k * n + i] * x[k];
    x[i] = s / F[(size_t)i * n + i];
  }
  search_dot = decrement = 0;
  for (int i = 0; i < n; ++i) {
    w.search[i] = -x[i];
    search_dot += x[i] * x[i];
    decrement += w.grad[i] * x[i];
  }
}

// ---- exact line search (iterative_search, mjwarp_linesearch.cu:81-375)
struct Row {
  int kind;   // 0 equality, 1 frictionloss, 2 inequality, 3 primary cone, 4 secondary cone
  T x, v, d, loss;
  T q0, q1, q2, u0, v0, uu, uv, vv, dm, mu;
  T cost0, t0, r0;
  int state0;
};

Point quadratic(T q1, T q2, T a) {
  T aq2 = a * q2;
  return {a * aq2 + a * q1, 2 * aq2 + q1, 2 * q2};
}
bool in_bracket(const Point& x, const Point& y) {
  return (x.slope < y.slope && y.slope < 0) || (x.slope > y.slope && y.slope > 0);
}

Point friction_point(const Row& r, T x) {
  T rf = safe_div(r.loss, r.d);
  if (-rf < x && x < rf) { T vd = r.v * r.d; return {0.5 * r.d * x * x, vd * x, r.v * vd}; }
  if (x <= -rf) return {r.loss * (-0.5 * rf - x), -r.loss * r.v, 0};
  return {r.loss * (-0.5 * rf + x), r.loss * r.v, 0};
}

Point evaluate_zero(const Row& r) {
  if (r.kind == 4) return {0, 0, 0};
  if (r.kind == 3) {
    if (r.state0 == 1) return {r.q0, r.q1, 2 * r.q2};
    if (r.state0 == 4) {
      T ti = 1 / r.t0, t1 = r.uv * ti, t2 = (r.vv - t1 * t1) * ti, r1 = r.v0 - r.mu * t1;
      return {r.cost0, r.dm * r.r0 * r1, r.dm * (r1 * r1 - r.mu * r.r0 * t2)};
    }
    return {0, 0, 0};
  }
  if (r.kind == 1) return friction_point(r, r.x);
  if (r.kind == 2 && r.x >= 0) return {0, 0, 0};
  T vd = r.v * r.d;
  return {0.5 * r.d * r.x * r.x, vd * r.x, r.v * vd};
}

Point cone_quadratic_shifted(const Row& r, T a, T n, T tsqr) {
  T aq2 = a * r.q2;
  T cost = a * (aq2 + r.q1);
  if (r.state0 == 4) { T bd = r.mu * r.u0 + r.t0; cost += 0.5 * r.dm * bd * bd; }
  else if (r.state0 == 0) cost = 0.5 * r.dm * (1 + r.mu * r.mu) * (n * n + std::max(tsqr, T(0)));
  return {cost, 2 * aq2 + r.q1, 2 * r.q2};
}

Point evaluate_shifted(const Row& r, T a) {
  if (r.kind == 4) return {0, 0, 0};
  if (r.kind == 3) {
    T n = r.u0 + a * r.v0, tsd = a * (2 * r.uv + a * r.vv), tsqr = r.uu + tsd;
    if (tsqr <= 0) {
      if (n < 0) return cone_quadratic_shifted(r, a, n, tsqr);
    } else {
      T t = std::sqrt(tsqr);
      if (n >= r.mu * t) {}
      else if (r.mu * n + t <= 0) return cone_quadratic_shifted(r, a, n, tsqr);
      else {
        T ti = 1 / t, t1 = (r.uv + a * r.vv) * ti, t2 = (r.vv - t1 * t1) * ti;
        T res = n - r.mu * t, r1 = r.v0 - r.mu * t1, cost;
        if (r.state0 == 4) {
          T td = tsd / (t + r.t0), rd = a * r.v0 - r.mu * td;
          cost = 0.5 * r.dm * rd * (2 * r.r0 + rd);
        } else if (r.state0 == 1) {
          T aq2 = a * r.q2, bd = r.mu * n + t;
          cost = a * (aq2 + r.q1) - 0.5 * r.dm * bd * bd;
        } else cost = 0.5 * r.dm * res * res;
        return {cost, r.dm * res * r1, r.dm * (r1 * r1 + res * (-r.mu * t2))};
      }
    }
    return {-r.cost0, 0, 0};
  }
  if (r.kind == 1) {
    Point p = friction_point(r, r.x + a * r.v);
    p.cost -= friction_point(r, r.x).cost;
    return p;
  }
  T quad0 = 0.5 * r.d * r.x * r.x;
  T cost0 = r.kind == 2 && r.x >= 0 ? 0 : quad0;
  if (r.kind == 2 && r.x + a * r.v >= 0) return {-cost0, 0, 0};
  T vd = r.v * r.d, h = r.v * vd, ah = a * h;
  return {a * (vd * r.x + 0.5 * ah) + (quad0 - cost0), vd * r.x + ah, h};
}

// returns alpha; sets improvement and the converged flag
T linesearch(const OrModel& m, World& w, T search_dot, T& improvement, bool& converged) {
  int nv = m.nv, R = w.nefc;
  const T kNoise = 8 * 1.1920929e-7;
  // Mv, Jv
  mul_m(m, w.M.data(), w.search.data(), w.Mv.data());
  for (int r = 0; r < R; ++r) {
    T s = 0;
    for (int i = 0; i < nv; ++i) s += w.J[(size_t)r * nv + i] * w.search[i];
    w.jv[r] = s;
  }
  T ratio = 1 / std::sqrt(m.opt_impratio);
  // elliptic cone quadratic coefficients per contact
  for (const Contact& ct : w.contacts) {
    int at = ct.efc_address;
    if (at < 0 || w.type[at] != EFC_ELLIPTIC) continue;
    T x = w.jaref[at], v = w.jv[at], d = w.D[at], vd = v * d;
    T q0 = 0.5 * x * x * d, q1 = vd * x, q2 = 0.5 * v * vd;
    T mu = ct.friction[0] * ratio;
    T u0 = x * mu, v0 = v * mu, uu = 0, uv = 0, vv = 0;
    for (int j = 1; j < ct.dim; ++j) {
      int t = at + j;
      T jvv = w.jv[t], ja = w.jaref[t], dj = w.D[t], djx = dj * ja;
      q0 += 0.5 * ja * djx; q1 += jvv * djx; q2 += 0.5 * jvv * dj * jvv;
      T f = ct.friction[j - 1], uj = ja * f, vj = jvv * f;
      uu += uj * uj; uv += uj * vj; vv += vj * vj;
    }
    int one = at + 1, two = at + 2;
    w.quad[3 * at] = q0; w.quad[3 * at + 1] = q1; w.quad[3 * at + 2] = q2;
    w.quad[3 * one] = u0; w.quad[3 * one + 1] = v0; w.quad[3 * one + 2] = uu;
    w.quad[3 * two] = uv; w.quad[3 * two + 1] = vv;
    T mu2 = mu * mu;
    w.quad[3 * two + 2] = d / (mu2 * (1 + mu2));
  }
  auto load = [&](int r) {
    Row x{};
    if (r < w.ne) x.kind = 0;
    else if (r < w.ne + w.nf) x.kind = 1;
    else if (w.type[r] != EFC_ELLIPTIC) x.kind = 2;
    else {
      const Contact& ct = w.contacts[w.id[r]];
      if (r != ct.efc_address) { x.kind = 4; return x; }
      x.kind = 3;
      int r1 = ct.efc_address + 1, r2 = ct.efc_address + 2;
      x.q0 = w.quad[3 * r]; x.q1 = w.quad[3 * r + 1]; x.q2 = w.quad[3 * r + 2];
      x.u0 = w.quad[3 * r1]; x.v0 = w.quad[3 * r1 + 1]; x.uu = w.quad[3 * r1 + 2];
      x.uv = w.quad[3 * r2]; x.vv = w.quad[3 * r2 + 1]; x.dm = w.quad[3 * r2 + 2];
      x.mu = ct.friction[0] * ratio;
      if (x.uu <= 0) { x.state0 = x.u0 < 0 ? 1 : 0; x.cost0 = x.state0 == 1 ? x.q0 : 0; }
      else {
        x.t0 = std::sqrt(x.uu);
        if (x.u0 >= x.mu * x.t0) x.state0 = 0;
        else if (x.mu * x.u0 + x.t0 <= 0) { x.state0 = 1; x.cost0 = x.q0; }
        else { x.state0 = 4; x.r0 = x.u0 - x.mu * x.t0; x.cost0 = 0.5 * x.dm * x.r0 * x.r0; }
      }
      return x;
    }
    x.x = w.jaref[r]; x.v = w.jv[r]; x.d = w.D[r];
    if (x.kind == 1) x.loss = w.frictionloss[r];
    return x;
  };
  T scale = m.meaninertia * nv;
  T gtol = std::max(m.opt_tolerance * m.opt_ls_tolerance * std::sqrt(search_dot) * scale, 1e-6);
  T g1 = 0, g2 = 0;
  for (int i = 0; i < nv; ++i) { g1 += w.search[i] * (w.Ma[i] - w.qfrc_smooth[i]); g2 += 0.5 * w.search[i] * w.Mv[i]; }
  for (int r = 0; r < w.ne; ++r) { T vd = w.jv[r] * w.D[r]; g1 += vd * w.jaref[r]; g2 += 0.5 * w.jv[r] * vd; }
  std::vector<Row> rows(R);
  for (int r = w.ne; r < R; ++r) rows[r] = load(r);
  Point rowsum{0, 0, 0};
  for (int r = w.ne; r < R; ++r) rowsum = rowsum + evaluate_zero(rows[r]);
  Point p0 = Point{0, g1, 2 * g2} + rowsum;
  Point delta{0, p0.slope, p0.curv};
  T q1abs = std::sqrt(2 * std::max(rowsum.cost, T(0)) * std::max(rowsum.curv, T(0))) + std::fabs(g1);
  T gacc = std::max(gtol, kNoise * q1abs), alpha = 0;
  improvement = 0;
  converged = std::fabs(p0.slope) < kNoise * q1abs;
  auto eval = [&](T a) {
    Point s{0, 0, 0};
    for (int r = w.ne; r < R; ++r) s = s + evaluate_shifted(rows[r], a);
    return quadratic(g1, g2, a) + s;
  };
  T ia = -safe_div(p0.slope, p0.curv);
  Point initial{0, 0, 0};
  if (!converged) {
    initial = eval(ia);
    if (std::fabs(initial.slope) < gacc && initial.cost < 0) { converged = true; alpha = ia; improvement = -initial.cost; }
  }
  if (!converged) {
    bool less = initial.slope < p0.slope;
    Point lo = less ? initial : delta, hi = less ? delta : initial;
    T la = less ? ia : 0, ha = less ? 0 : ia;
    for (int it = 0; it < m.opt_ls_iterations; ++it) {
      T ln = la - safe_div(lo.slope, lo.curv), hn = ha - safe_div(hi.slope, hi.curv), ma = 0.5 * (la + ha);
      Point nlo = eval(ln), nhi = eval(hn), mid = eval(ma);
      bool cl = std::fabs(nlo.slope) < gacc && nlo.cost < 0;
      bool ch = std::fabs(nhi.slope) < gacc && nhi.cost < 0;
      bool cm = std::fabs(mid.slope) < gacc && mid.cost < 0;
      bool any = cl || ch || cm, swl = false, swh = false;
      if (any) {
        Point best{1e10, 0, 0};
        T ba = 0;
        if (cl && nlo.cost < best.cost) { best = nlo; ba = ln; }
        if (ch && nhi.cost < best.cost) { best = nhi; ba = hn; }
        if (cm && mid.cost < best.cost) { best = mid; ba = ma; }
        lo = hi = best; la = ha = ba;
      } else {
        bool s = in_bracket(lo, nlo);
        if (s) { lo = nlo; la = ln; } swl |= s;
        s = in_bracket(lo, mid);
        if (s) { lo = mid; la = ma; } swl |= s;
        s = in_bracket(lo, nhi);
        if (s) { lo = nhi; la = hn; } swl |= s;
        s = in_bracket(hi, nhi) || (hi.slope < 0 && nhi.slope > 0);
        if (s) { hi = nhi; ha = hn; } swh |= s;
        s = in_bracket(hi, mid);
        if (s) { hi = mid; ha = ma; } swh |= s;
        s = in_bracket(hi, nlo);
        if (s) { hi = nlo; ha = ln; } swh |= s;
      }
      bool done = any || (!swl && !swh) || (lo.cost < 0 && lo.slope < 0 && lo.slope > -gtol) ||
                  (hi.cost < 0 && hi.slope > 0 && hi.slope < gtol);
      if (lo.cost < 0 || hi.cost < 0) {
        bool bl = lo.cost < hi.cost;
        alpha = bl ? la : ha;
        improvement = -(bl ? lo.cost : hi.cost);
      }
      if (done) { converged = true; break; }
    }
  }
  for (int i = 0; i < nv; ++i) { w.qacc[i] += alpha * w.search[i]; w.Ma[i] += alpha * w.Mv[i]; }
  for (int r = 0; r < R; ++r) w.jaref[r] += alpha * w.jv[r];
  return alpha;
}

}  // namespace

void mul_m(const OrModel& m, const T* M, const T* x, T* y) {
  for (int t = 0; t < m.ntree; ++t) {
    int n = m.tree_dofnum[t], a = m.tree_dofadr[t];
    const T* blk = M + m.tree_madr[t];
    for (int i = 0; i < n; ++i) {
      T s = 0;
      for (int j = 0; j < n; ++j) s += blk[i * n + j] * x[a + j];
      y[a + i] = s;
    }
  }
}

// Dense Newton with exact line search (MJWarp solver as run by the reference, see file header).
void newton(const OrModel& m, World& w, const T* warmstart) {
  int nv = m.nv, R = w.nefc;
  w.niter = 0;
  w.overflow &= ~(MX_OVERFLOW_ITERATIONS | MX_OVERFLOW_LS_ITERATIONS);
  bool warm = !(m.opt_disableflags & (1 << 8));
  for (int i = 0; i < nv; ++i) w.qacc[i] = (warm && R > 0) ? warmstart[i] : w.qacc_smooth[i];
  if (R == 0) {
    std::fill(w.qfrc_constraint.begin(), w.qfrc_constraint.end(), 0.0);
    for (int i = 0; i < nv; ++i) w.qacc[i] = w.qacc_smooth[i];
    return;
  }
  mul_m(m, w.M.data(), w.qacc.data(), w.Ma.data());
  for (int r = 0; r < R; ++r) {
    T s = 0;
    for (int i = 0; i < nv; ++i) s += w.J[(size_t)r * nv + i] * w.qacc[i];
    w.jaref[r] = s - w.aref[r];
  }
  T search_dot, decrement;
  gradient(m, w);
  hessian(m, w);
  direction(m, w, search_dot, decrement);
  if (m.opt_iterations <= 0) return;
  T scale = m.meaninertia * nv;
  for (;;) {
    T improvement;
    bool ls_ok;
    T alpha = linesearch(m, w, search_dot, improvement, ls_ok);
    if (!ls_ok) w.overflow |= MX_OVERFLOW_LS_ITERATIONS;
    gradient(m, w);
    hessian(m, w);
    direction(m, w, search_dot, decrement);
    int iterations = ++w.niter;
    T grad_dot = 0;
    for (int i = 0; i < nv; ++i) grad_dot += w.grad[i] * w.grad[i];
    T imp = improvement / scale, g = std::sqrt(grad_dot) / scale, mi = 0.5 * decrement / scale;
    T tol = m.opt_tolerance;
    bool done = alpha == 0 || (imp > 0 && imp < tol) || g < tol || mi < tol;
    if (done || iterations == m.opt_iterations) {
      if (!done) w.overflow |= MX_OVERFLOW_ITERATIONS;
      break;
    }
  }
}

}  // namespace orc
