// ORACLE — test infrastructure only.
//
// A CPU (OpenMP) restatement of the reference's event-transport loops, used as the checker for the HIP
// library and as the timed CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
// leg may load this library; the product path (x_amd) never does.
//
// Each function follows csrc/atl_cpu.cpp of the reference (file:line cited per function): same loop order,
// same float arithmetic (no FMA: this file is built with plain `g++ -O3 -fopenmp` for x86-64 baseline,
// whose SSE2 code has no fused multiply-add), same OpenMP schedules, `omp atomic` scatters and the double
// accumulator of the pair forward.  The pair forward additionally reports n_i, the number of visited
// (contributing) pairs per anchor, which the reference does not output.
//
// Parity pins (tests/test_oracle.py): fp64 brute force of the defining sums, adjoint identities
// <splat(w), G> = <w, gather(G)>, mass conservation, finite differences, and the reference's own
// known-answer tests (tests/test_ops.py:90-100).
#include <cmath>
#include <cstdint>
#include <omp.h>

namespace {

// Up to four in-image bilinear corners of (x, y): csrc/atl_cpu.cpp:17-33.
template <typename F>
inline void corners(float x, float y, int64_t H, int64_t W, F&& f) {
  const float fx = std::floor(x), fy = std::floor(y);
  const int64_t x0 = (int64_t)fx, y0 = (int64_t)fy;
  const float ax = x - fx, ay = y - fy;
  const float wx[2] = {1.f - ax, ax};
  const float wy[2] = {1.f - ay, ay};
  const float dw[2] = {-1.f, 1.f};
  for (int j = 0; j < 2; ++j) {
    const int64_t yy = y0 + j;
    if (yy < 0 || yy >= H) continue;
    for (int i = 0; i < 2; ++i) {
      const int64_t xx = x0 + i;
      if (xx < 0 || xx >= W) continue;
      f(yy, xx, wx[i] * wy[j], dw[i] * wy[j], wx[i] * dw[j]);
    }
  }
}

struct PairView {
  const float *SY, *SV, *ST, *AX, *AT, *SC;
  const int64_t *SID, *CS, *AC, *AID;
  int64_t S, GH, GW;
  float h, tau, cut;
};

// Walk of the 3x3 cell neighbourhood of anchor i with the reference's pair tests:
// csrc/atl_cpu.cpp:176-200.
template <typename Visit>
inline void pairs_of(int64_t i, const PairView& p, Visit&& visit) {
  const float xi = p.AX[2 * i], yi = p.AX[2 * i + 1], ti = p.AT[i];
  const int64_t g = p.AC[3 * i], cx = p.AC[3 * i + 1], cy = p.AC[3 * i + 2], id = p.AID[i];
  const float cs = p.SC[g % p.S];
  const float r2max = p.cut * p.cut * p.h * p.h;
  const float inv2h2 = 1.f / (2.f * p.h * p.h);
  const int64_t ylo = cy - 1 < 0 ? 0 : cy - 1, yhi = cy + 1 > p.GH - 1 ? p.GH - 1 : cy + 1;
  const int64_t xlo = cx - 1 < 0 ? 0 : cx - 1, xhi = cx + 1 > p.GW - 1 ? p.GW - 1 : cx + 1;
  for (int64_t yy = ylo; yy <= yhi; ++yy) {
    for (int64_t xx = xlo; xx <= xhi; ++xx) {
      const int64_t cell = (g * p.GH + yy) * p.GW + xx;
      for (int64_t k = p.CS[cell]; k < p.CS[cell + 1]; ++k) {
        if (p.SID[k] == id) continue;
        const float dt = ti - p.ST[k];
        if (std::fabs(dt) > p.tau) continue;
        const float rx = xi - (p.SY[2 * k] + p.SV[2 * k] * (ti - cs));
        const float ry = yi - (p.SY[2 * k + 1] + p.SV[2 * k + 1] * (ti - cs));
        const float d2 = rx * rx + ry * ry;
        if (d2 > r2max) continue;
        visit(k, rx, ry, dt, std::exp(-d2 * inv2h2));
      }
    }
  }
}

}  // namespace

extern "C" {

int oracle_num_threads(void) { return omp_get_max_threads(); }

// csrc/atl_cpu.cpp:38-56
void oracle_splat_bilinear_fwd(const float* P, const float* Wt, const int64_t* Bi, int64_t N, int64_t B, int64_t H,
                               int64_t W, float* I) {
  (void)B;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const float wn = Wt[n];
    if (wn == 0.f) continue;
    float* img = I + Bi[n] * H * W;
    corners(P[2 * n], P[2 * n + 1], H, W, [&](int64_t yy, int64_t xx, float c, float, float) {
#pragma omp atomic
      img[yy * W + xx] += wn * c;
    });
  }
}

// csrc/atl_cpu.cpp:58-76
void oracle_splat_bilinear_bwd(const float* G, const float* P, const float* Wt, const int64_t* Bi, int64_t N,
                               int64_t H, int64_t W, float* GP, float* GWt) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const float* g = G + Bi[n] * H * W;
    float sx = 0.f, sy = 0.f, sw = 0.f;
    corners(P[2 * n], P[2 * n + 1], H, W, [&](int64_t yy, int64_t xx, float c, float dcx, float dcy) {
      const float v = g[yy * W + xx];
      sw += v * c;
      sx += v * dcx;
      sy += v * dcy;
    });
    GWt[n] = sw;
    GP[2 * n] = Wt[n] * sx;
    GP[2 * n + 1] = Wt[n] * sy;
  }
}

// csrc/atl_cpu.cpp:79-104
void oracle_splat_gauss_fwd(const float* P, const float* Wt, const int64_t* Bi, int64_t N, int64_t H, int64_t W,
                            double sigma, int64_t R, float* I) {
  const float inv2s2 = 1.f / (2.f * (float)(sigma * sigma));
  const float norm = 1.f / (2.f * (float)M_PI * (float)(sigma * sigma));
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const float wn = Wt[n] * norm;
    if (wn == 0.f) continue;
    const float x = P[2 * n], y = P[2 * n + 1];
    const int64_t cx = (int64_t)std::lround(x), cy = (int64_t)std::lround(y);
    float* img = I + Bi[n] * H * W;
    const int64_t ylo = cy - R < 0 ? 0 : cy - R, yhi = cy + R > H - 1 ? H - 1 : cy + R;
    const int64_t xlo = cx - R < 0 ? 0 : cx - R, xhi = cx + R > W - 1 ? W - 1 : cx + R;
    for (int64_t yy = ylo; yy <= yhi; ++yy) {
      const float dy = (float)yy - y;
      for (int64_t xx = xlo; xx <= xhi; ++xx) {
        const float dx = (float)xx - x;
        const float v = wn * std::exp(-(dx * dx + dy * dy) * inv2s2);
#pragma omp atomic
        img[yy * W + xx] += v;
      }
    }
  }
}

// csrc/atl_cpu.cpp:106-131
void oracle_splat_gauss_bwd(const float* G, const float* P, const float* Wt, const int64_t* Bi, int64_t N, int64_t H,
                            int64_t W, double sigma, int64_t R, float* GP, float* GWt) {
  const float s2 = (float)(sigma * sigma);
  const float inv2s2 = 1.f / (2.f * s2), norm = 1.f / (2.f * (float)M_PI * s2);
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const float x = P[2 * n], y = P[2 * n + 1];
    const int64_t cx = (int64_t)std::lround(x), cy = (int64_t)std::lround(y);
    const float* g = G + Bi[n] * H * W;
    float sw = 0.f, sx = 0.f, sy = 0.f;
    const int64_t ylo = cy - R < 0 ? 0 : cy - R, yhi = cy + R > H - 1 ? H - 1 : cy + R;
    const int64_t xlo = cx - R < 0 ? 0 : cx - R, xhi = cx + R > W - 1 ? W - 1 : cx + R;
    for (int64_t yy = ylo; yy <= yhi; ++yy) {
      const float dy = (float)yy - y;
      for (int64_t xx = xlo; xx <= xhi; ++xx) {
        const float dx = (float)xx - x;
        const float gk = norm * std::exp(-(dx * dx + dy * dy) * inv2s2) * g[yy * W + xx];
        sw += gk;
        sx += gk * dx / s2;
        sy += gk * dy / s2;
      }
    }
    GWt[n] = sw;
    GP[2 * n] = Wt[n] * sx;
    GP[2 * n + 1] = Wt[n] * sy;
  }
}

// csrc/atl_cpu.cpp:134-149
void oracle_gather_bilinear_fwd(const float* I, const float* P, const int64_t* Bi, int64_t N, int64_t H, int64_t W,
                                float* O) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const float* img = I + Bi[n] * H * W;
    float s = 0.f;
    corners(P[2 * n], P[2 * n + 1], H, W,
            [&](int64_t yy, int64_t xx, float c, float, float) { s += c * img[yy * W + xx]; });
    O[n] = s;
  }
}

// csrc/atl_cpu.cpp:151-172
void oracle_gather_bilinear_bwd(const float* GV, const float* I, const float* P, const int64_t* Bi, int64_t N,
                                int64_t H, int64_t W, float* GI, float* GP) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const float g = GV[n];
    const float* img = I + Bi[n] * H * W;
    float* gimg = GI + Bi[n] * H * W;
    float sx = 0.f, sy = 0.f;
    corners(P[2 * n], P[2 * n + 1], H, W, [&](int64_t yy, int64_t xx, float c, float dcx, float dcy) {
      const float v = img[yy * W + xx];
      sx += dcx * v;
      sy += dcy * v;
#pragma omp atomic
      gimg[yy * W + xx] += g * c;
    });
    GP[2 * n] = g * sx;
    GP[2 * n + 1] = g * sy;
  }
}

// csrc/atl_cpu.cpp:203-222, plus the instrumented neighbour count n_i (visits per anchor; may be null).
void oracle_ats_pair_fwd(const float* SY, const float* SV, const float* ST, const int64_t* SID, const int64_t* CS,
                         const float* AX, const float* AT, const int64_t* AC, const int64_t* AID, const float* SC,
                         int64_t M, int64_t S, int64_t GH, int64_t GW, double h, double tau, double cut, float* O,
                         int64_t* count) {
  const PairView p{SY, SV, ST, AX, AT, SC, SID, CS, AC, AID, S, GH, GW, (float)h, (float)tau, (float)cut};
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t i = 0; i < M; ++i) {
    double acc = 0.0;
    int64_t n = 0;
    pairs_of(i, p, [&](int64_t, float, float, float, float k) {
      acc += k;
      ++n;
    });
    O[i] = (float)acc;
    if (count) count[i] = n;
  }
}

// csrc/atl_cpu.cpp:224-253.  GV (N,2) must be zero-filled by the caller.
void oracle_ats_pair_bwd(const float* G, const float* SY, const float* SV, const float* ST, const int64_t* SID,
                         const int64_t* CS, const float* AX, const float* AT, const int64_t* AC, const int64_t* AID,
                         const float* SC, int64_t M, int64_t S, int64_t GH, int64_t GW, double h, double tau,
                         double cut, float* GV) {
  const PairView p{SY, SV, ST, AX, AT, SC, SID, CS, AC, AID, S, GH, GW, (float)h, (float)tau, (float)cut};
  const float invh2 = 1.f / (float)(h * h);
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t i = 0; i < M; ++i) {
    const float gi = G[i];
    if (gi == 0.f) continue;
    pairs_of(i, p, [&](int64_t k, float rx, float ry, float dt, float kern) {
      const float f = gi * kern * dt * invh2;
      const int64_t j = SID[k];
#pragma omp atomic
      GV[2 * j] += f * rx;
#pragma omp atomic
      GV[2 * j + 1] += f * ry;
    });
  }
}

// Backward of the trajectory pair sums (no reference implementation; the definition's gradient in the loop form
// of csrc/atl_cpu.cpp:224-253): per visited pair (anchor i, entry k of source j in slice s), dL/dy = g k r / h^2
// and dL/dv = g k r at / h^2 (at = t_i - c_s), chained through y = p + sum_c coef_c tab[s][c] and
// v = sum_c coef_c tab[s][K + c] into GP (N,2) and GC (N, 2K, channels [y_1..y_K, x_1..x_K]); float64
// accumulators, zero-filled by the caller.
void oracle_ats_pair_bwd_traj(const float* G, const float* SY, const float* SV, const float* ST, const int64_t* SID,
                              const int64_t* CS, const float* AX, const float* AT, const int64_t* AC,
                              const int64_t* AID, const float* SC, int64_t M, int64_t S, int64_t GH, int64_t GW,
                              double h, double tau, double cut, const float* TAB, int64_t K, double* GP,
                              double* GC) {
  const PairView p{SY, SV, ST, AX, AT, SC, SID, CS, AC, AID, S, GH, GW, (float)h, (float)tau, (float)cut};
  const double invh2 = 1.0 / (h * h);
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t i = 0; i < M; ++i) {
    const double gi = G[i];
    if (gi == 0.0) continue;
    const int64_t s = AC[3 * i] % S;
    const double at = (double)(AT[i] - SC[s]);
    const float* row = TAB + s * 2 * K;
    pairs_of(i, p, [&](int64_t k, float rx, float ry, float, float kern) {
      const double f = gi * kern * invh2;
      const int64_t j = SID[k];
#pragma omp atomic
      GP[2 * j] += f * rx;
#pragma omp atomic
      GP[2 * j + 1] += f * ry;
      for (int64_t c = 0; c < K; ++c) {
        const double wy = row[c] + at * row[K + c];
#pragma omp atomic
        GC[j * 2 * K + c] += f * ry * wy;
#pragma omp atomic
        GC[j * 2 * K + K + c] += f * rx * wy;
      }
    });
  }
}

// csrc/atl_cpu.cpp:256-286
void oracle_voxel_grid(const float* P, const float* T, const float* Pol, const int64_t* Bi, int64_t N, int64_t C,
                       int64_t H, int64_t W, float* V) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const float x = P[2 * n], y = P[2 * n + 1], tn = T[n] * (float)(C - 1);
    const int64_t x0 = (int64_t)std::floor(x), y0 = (int64_t)std::floor(y), t0 = (int64_t)std::floor(tn);
    for (int dt = 0; dt < 2; ++dt) {
      const int64_t tt = t0 + dt;
      if (tt < 0 || tt >= C) continue;
      const float wt = 1.f - std::fabs((float)tt - tn);
      for (int dy = 0; dy < 2; ++dy) {
        const int64_t yy = y0 + dy;
        if (yy < 0 || yy >= H) continue;
        const float wy = 1.f - std::fabs((float)yy - y);
        for (int dx = 0; dx < 2; ++dx) {
          const int64_t xx = x0 + dx;
          if (xx < 0 || xx >= W) continue;
          const float wx = 1.f - std::fabs((float)xx - x);
#pragma omp atomic
          V[((Bi[n] * C + tt) * H + yy) * W + xx] += Pol[n] * wt * wy * wx;
        }
      }
    }
  }
}

}  // extern "C"

extern "C" {
// vmax of build_pair_plan (atl/ops/functional.py:139): max_j ||v_j|| as torch's CPU vector norm evaluates it
// on AVX2/AVX-512 hosts, sqrt(fma(vy, vy, vx*vx)) in fp32 (the fused form was identified by comparing
// torch.linalg.vector_norm against candidate roundings on 1M random vectors: zero mismatches).
float oracle_vmax(const float* V, int64_t N) {
  float m = 0.f;
  for (int64_t j = 0; j < N; ++j) {
    const float vx = V[2 * j], vy = V[2 * j + 1];
    const float n = std::sqrt(std::fmaf(vy, vy, vx * vx));
    if (n > m) m = n;
  }
  return m;
}
}  // extern "C"
