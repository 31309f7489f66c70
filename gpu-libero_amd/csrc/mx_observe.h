// Observation sampling: an ordered robosuite observable plan evaluated per world by one wavefront
// (reference gpu/cuda/fp32/fused_observations.cu:39-168 pack_and_sample).  The clocks run one lane
// per spec; the specs then execute in plan order (a spec may read earlier specs' values): gathers
// and cos / sin one lane per value, the pose operations on one lane.  The values, the sampling
// state and the aside quaternions stay in the plan's device arrays; a wave barrier orders each
// spec's stores before the next spec's loads.
#pragma once
#include <hip/hip_runtime.h>
#include "../../include/mx_physics.h"

namespace MX_NS {

typedef const __attribute__((address_space(4))) MxObsPlan KObsPlan;

// robosuite quat2mat of a quaternion (x, y, z, w): rescaled by sqrt(2 / |q|^2), identity below
// 4 * eps64 (the reference's FP32 convention, fused_observations.cu:10-20)
__device__ inline void obs_quat_mat(const float* q, float* r) {
  const float w = q[3], x = q[0], y = q[1], z = q[2];
  const float n = w * w + x * x + y * y + z * z;
  for (int i = 0; i < 9; ++i) r[i] = (i % 4 == 0) ? 1.f : 0.f;
  if (n < float(4.0 * 2.220446049250313e-16)) return;
  const float s = sqrtf(2.f / n);
  const float W = w * s, X = x * s, Y = y * s, Z = z * s;
  r[0] = 1.f - Y * Y - Z * Z; r[1] = X * Y - Z * W;       r[2] = X * Z + Y * W;
  r[3] = X * Y + Z * W;       r[4] = 1.f - X * X - Z * Z; r[5] = Y * Z - X * W;
  r[6] = X * Z - Y * W;       r[7] = Y * Z + X * W;       r[8] = 1.f - X * X - Y * Y;
}

// robosuite mat2quat: the quaternion (x, y, z, w), w >= 0, of a rotation matrix.  robosuite takes
// the dominant eigenvector of Bar-Itzhack's symmetric 4x4 K; for a rotation matrix that is the
// quaternion Shepperd's method gives in closed form from the largest of (trace, m00, m11, m22).
__device__ inline void obs_mat_quat(const float* m, float* q) {
  const float tr = m[0] + m[4] + m[8];
  float x, y, z, w;
  if (tr >= m[0] && tr >= m[4] && tr >= m[8]) {
    const float s = 2.f * sqrtf(fmaxf(1.f + tr, 1e-30f));
    w = 0.25f * s; x = (m[7] - m[5]) / s; y = (m[2] - m[6]) / s; z = (m[3] - m[1]) / s;
  } else if (m[0] >= m[4] && m[0] >= m[8]) {
    const float s = 2.f * sqrtf(fmaxf(1.f + m[0] - m[4] - m[8], 1e-30f));
    x = 0.25f * s; w = (m[7] - m[5]) / s; y = (m[1] + m[3]) / s; z = (m[2] + m[6]) / s;
  } else if (m[4] >= m[8]) {
    const float s = 2.f * sqrtf(fmaxf(1.f + m[4] - m[0] - m[8], 1e-30f));
    y = 0.25f * s; w = (m[2] - m[6]) / s; x = (m[1] + m[3]) / s; z = (m[5] + m[7]) / s;
  } else {
    const float s = 2.f * sqrtf(fmaxf(1.f + m[8] - m[0] - m[4], 1e-30f));
    z = 0.25f * s; w = (m[3] - m[1]) / s; x = (m[2] + m[6]) / s; y = (m[5] + m[7]) / s;
  }
  const float n = rsqrtf(x * x + y * y + z * z + w * w), sg = w < 0.f ? -n : n;
  q[0] = x * sg; q[1] = y * sg; q[2] = z * sg; q[3] = w * sg;
}

// Orders the calling wavefront's accesses between two samples.  The call is made by one wave (its
// workgroup may hold a second wave that does not sample), so the barrier is the wave's own: its
// memory operations complete in order, and the fences keep the compiler from moving accesses
// across the barrier.
__device__ __forceinline__ void obs_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One sampling call for world w by all lanes of its wavefront.  src(code) returns a gathered
// source value (code = MX_OBS_SRC << 24 | element; 0 for an element outside its field).
template <class Src>
__device__ void obs_sample(KObsPlan& p, size_t w, int lane, float dt, int force, Src src) {
  const int ns = p.nspec, width = p.width;
  float* cache = p.cache + w * width;
  float* obs = p.observed + w * width;
  float* side = p.sidequat + w * width;
  int* present = p.present + w * ns;
  unsigned long long act[2] = {0ull, 0ull};
#pragma unroll
  for (int half = 0; half < 2; ++half) {   // clocks, one lane per spec
    const int s = lane + 64 * half;
    bool take = false;
    if (s < ns) {
      const size_t at = w * ns + s;
      p.events[at] = 0;
      if (p.enabled[s]) {
        const int sampled = p.sampled[at];
        const float elapsed = p.elapsed[at] + dt, period = p.period[s];
        const bool due = elapsed >= period;
        take = (!sampled && period >= elapsed) || force || (due && !sampled);
        p.elapsed[at] = due ? fmodf(elapsed, period) : elapsed;
        p.sampled[at] = due ? 0 : (take ? 1 : sampled);
      }
    }
    act[half] = __ballot(take);
  }
  if (!(act[0] | act[1])) return;
  for (int half = 0; half < 2; ++half)
    for (unsigned long long bits = act[half]; bits; bits &= bits - 1) {
      const int s = 64 * half + __ffsll((long long)bits) - 1;
      const int at = p.offset[s], n = p.size[s], op = p.op[s];
      if (at < 0 || n < 0 || at + n > width) continue;     // a malformed spec samples nothing
      auto here = [&](int i) {
        const int dep = p.presence[3 * s + i];
        return dep >= 0 && dep < ns && present[dep] != 0;
      };
      if (op <= MX_OBS_SIN) {
        const int d0 = p.dep0[s];
        const bool dep = op == MX_OBS_GATHER || here(0);
        for (int j = lane; j < n; j += 64) {
          float v = 0.f;
          if (op == MX_OBS_GATHER) v = src(p.indices[p.index_offset[s] + j]);
          else if (dep && d0 >= 0 && d0 + j < width) v = op == MX_OBS_COS ? cosf(cache[d0 + j]) : sinf(cache[d0 + j]);
          cache[at + j] = v;
          obs[at + j] = v;
        }
      } else if (lane == 0) {
        const int d0 = p.dep0[s], d1 = p.dep1[s], d2 = p.dep2[s];
        for (int j = 0; j < n; ++j) cache[at + j] = 0.f;
        if (op == MX_OBS_INVERSE_POSE && n >= 16) {
          if (!here(0) || !here(1) || d0 < 0 || d0 + 3 > width || d1 < 0 || d1 + 4 > width) {
            for (int r = 0; r < 4; ++r) cache[at + 5 * r] = 1.f;
          } else {
            float R[9];
            obs_quat_mat(cache + d1, R);
            for (int r = 0; r < 3; ++r) {   // [R^T, -R^T p; 0 0 0 1]
              float t = 0.f;
              for (int k = 0; k < 3; ++k) {
                cache[at + 4 * r + k] = R[3 * k + r];
                t -= R[3 * k + r] * cache[d0 + k];
              }
              cache[at + 4 * r + 3] = t;
            }
            cache[at + 15] = 1.f;
          }
        } else if (op == MX_OBS_RELATIVE_POS && n >= 3) {
          if (here(0) && here(1) && here(2) && d0 >= 0 && d0 + 3 <= width && d1 >= 0 && d1 + 4 <= width &&
              d2 >= 0 && d2 + 16 <= width) {
            float Ro[9], Rr[9];
            const float* T = cache + d2;
            obs_quat_mat(cache + d1, Ro);
            for (int r = 0; r < 3; ++r) {
              float t = T[4 * r + 3];
              for (int k = 0; k < 3; ++k) {
                t += T[4 * r + k] * cache[d0 + k];
                Rr[3 * r + k] = T[4 * r] * Ro[k] + T[4 * r + 1] * Ro[3 + k] + T[4 * r + 2] * Ro[6 + k];
              }
              cache[at + r] = t;
            }
            if (at + 4 <= width) obs_mat_quat(Rr, side + at);
          }
        } else if (op == MX_OBS_RELATIVE_QUAT && n >= 4) {
          if (here(0) && d0 >= 0 && d0 + 4 <= width)
            for (int k = 0; k < 4; ++k) cache[at + k] = side[d0 + k];
        }
        for (int j = 0; j < n; ++j) obs[at + j] = cache[at + j];
      }
      if (lane == 0) {
        present[s] = 1;
        p.events[w * ns + s] = 1;
      }
      obs_wave_sync();
    }
}

}  // namespace MX_NS
