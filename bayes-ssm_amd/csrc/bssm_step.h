// Per-token forward update shared by the gfx950 recurrence kernels
// (equation reference: bayes_ssm/bayesian_layer.py:207-251).
#pragma once

#include "bssm_recurrence.h"

namespace bssm {

// Fixed-dynamics constants (bayes_ssm/bayesian_layer.py:366-369,
// persistent_bayes_chunked_d4m8.cu:212-217).
constexpr float kFixedDecay = 0.97f;
constexpr float kFixedProcess = 0.1f;
constexpr float kFixedObservation = 1.0f;

// u (or any per-row quantity) from its row owners to every lane of the group.
template <int D, int M, int G, int R = 0>
__device__ __forceinline__ void gather_rows(const OwnRowVec<D, M, G>& own, float (&all)[D],
                                            int lane) {
  using L = Layout<D, M, G>;
  if constexpr (R < D) {
    all[R] = group_bcast<G, L::owner(R)>(own[L::slot(R)], lane);
    gather_rows<D, M, G, R + 1>(own, all, lane);
  }
}

// Per-lane recurrent belief.
template <int D, int M, int G>
struct Belief {
  using L = Layout<D, M, G>;
  float P[L::RPL][D];   // own covariance rows
  float Mv[D][L::CPL];  // all rows, own value columns
};

// Token inputs as seen by one lane.
template <int D, int M, int G>
struct TokenIn {
  using L = Layout<D, M, G>;
  float k[D], d[D];
  float k_own[L::RPL], d_own[L::RPL];
  float v[L::CPL];
  float p, r;
};

// Tile pointers of one sequence (already offset by the sequence slot).
struct SeqTile {
  const float* k;
  const float* d;
  const float* v;
  const float* p;
  const float* r;
};

template <int D, int M, int G, bool FIXED>
__device__ __forceinline__ void read_token(TokenIn<D, M, G>& in, const SeqTile& st, int tt, int g,
                                           bool need_v) {
  using L = Layout<D, M, G>;
#pragma unroll
  for (int j = 0; j < D; ++j) in.k[j] = st.k[tt * D + j];
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj) in.k_own[jj] = st.k[tt * D + L::row(g, jj)];
  if constexpr (FIXED) {
#pragma unroll
    for (int j = 0; j < D; ++j) in.d[j] = kFixedDecay;
#pragma unroll
    for (int jj = 0; jj < L::RPL; ++jj) in.d_own[jj] = kFixedDecay;
    in.p = kFixedProcess;
    in.r = kFixedObservation;
  } else {
#pragma unroll
    for (int j = 0; j < D; ++j) in.d[j] = st.d[tt * D + j];
#pragma unroll
    for (int jj = 0; jj < L::RPL; ++jj) in.d_own[jj] = st.d[tt * D + L::row(g, jj)];
    in.p = st.p[tt];
    in.r = st.r[tt];
  }
  if (need_v) {
#pragma unroll
    for (int c = 0; c < L::CPL; ++c) in.v[c] = st.v[tt * M + g * L::CPL + c];
  }
}

// What one forward step leaves for the reverse pass.
template <int D, int M, int G>
struct StepOut {
  using L = Layout<D, M, G>;
  float u[D];           // gathered u = P' k
  float u_own[L::RPL];  // own rows of u
  float s;              // unclamped innovation variance r + k.u
  float e[L::CPL];      // own innovations
};

// One forward token update.  `eye[jj][j]` is 1 where row(g, jj) == j.
template <int D, int M, int G>
__device__ __forceinline__ void forward_step(Belief<D, M, G>& b, const TokenIn<D, M, G>& in,
                                             const RowsArr<D, M, G>& eye, float floor,
                                             int lane, StepOut<D, M, G>& o) {
  using L = Layout<D, M, G>;
  float Pb[L::RPL][D];
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj) {
    float acc = in.p * in.k_own[jj];
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const float dp = (in.d_own[jj] * in.d[j]) * b.P[jj][j];
      Pb[jj][j] = fmaf(in.p, eye[jj][j], dp);
      acc = fmaf(dp, in.k[j], acc);
    }
    o.u_own[jj] = acc;
  }
  gather_rows<D, M, G>(o.u_own, o.u, lane);
  float s = in.r;
#pragma unroll
  for (int j = 0; j < D; ++j) s = fmaf(in.k[j], o.u[j], s);
  o.s = s;
  const float beta = fast_rcp(fmaxf(s, floor));
  float wk[D], bu[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    wk[j] = in.d[j] * in.k[j];
    bu[j] = beta * o.u[j];
  }
#pragma unroll
  for (int c = 0; c < L::CPL; ++c) {
    float e = in.v[c];
#pragma unroll
    for (int i = 0; i < D; ++i) e = fmaf(-b.Mv[i][c], wk[i], e);
    o.e[c] = e;
#pragma unroll
    for (int i = 0; i < D; ++i) b.Mv[i][c] = fmaf(bu[i], e, in.d[i] * b.Mv[i][c]);
  }
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj)
#pragma unroll
    for (int j = 0; j < D; ++j) b.P[jj][j] = fmaf(-beta, o.u_own[jj] * o.u[j], Pb[jj][j]);
}

template <int D, int M, int G>
__device__ __forceinline__ void init_eye(RowsArr<D, M, G>& eye, int g) {
  using L = Layout<D, M, G>;
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj)
#pragma unroll
    for (int j = 0; j < D; ++j) eye[jj][j] = (L::row(g, jj) == j) ? 1.f : 0.f;
}

template <int D, int M, int G>
__device__ __forceinline__ void load_belief(Belief<D, M, G>& b, const float* mean, const float* cov, int g,
                                            bool active) {
  using L = Layout<D, M, G>;
#pragma unroll
  for (int i = 0; i < D; ++i)
#pragma unroll
    for (int c = 0; c < L::CPL; ++c) b.Mv[i][c] = active ? mean[i * M + g * L::CPL + c] : 0.f;
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj)
#pragma unroll
    for (int j = 0; j < D; ++j)
      b.P[jj][j] = active ? cov[L::row(g, jj) * D + j] : (L::row(g, jj) == j ? 1.f : 0.f);
}

template <int D, int M, int G>
__device__ __forceinline__ void store_belief(const Belief<D, M, G>& b, float* mean, float* cov, int g) {
  using L = Layout<D, M, G>;
#pragma unroll
  for (int i = 0; i < D; ++i)
#pragma unroll
    for (int c = 0; c < L::CPL; ++c) mean[i * M + g * L::CPL + c] = b.Mv[i][c];
  if (L::row_writer(g)) {
#pragma unroll
    for (int jj = 0; jj < L::RPL; ++jj)
#pragma unroll
      for (int j = 0; j < D; ++j) cov[L::row(g, jj) * D + j] = b.P[jj][j];
  }
}

__device__ __forceinline__ int tile_len(int64_t t, int64_t t0, int tile) {
  return static_cast<int>((t - t0) < tile ? (t - t0) : tile);
}

// Everything the reverse of one token needs besides the token inputs.
template <int D, int M, int G>
struct RevIn {
  using L = Layout<D, M, G>;
  float q[D];
  float gy[L::CPL];
  float beta, s;              // 1/max(s, floor) and the unclamped s
  float u[D], u_own[L::RPL];  // u = P' k
  float e[L::CPL];            // own innovations
  float mp[D][L::CPL];        // d * M_prev (own columns)
  float Mprev[D][L::CPL];     // M_prev (own columns)
  float Pb[L::RPL][D];        // P' rows
  float Pprev[L::RPL][D];     // covariance rows before the token
};

template <int D, int M, int G>
struct RevOut {
  using L = Layout<D, M, G>;
  float gk_own[L::RPL], gq_own[L::RPL], gd_own[L::RPL];
  float gv[L::CPL];
  float gp, gr;
};

// Reverse of one token.  Carried adjoints: gM = dL/dM (own columns) and
// Gs = sym(dL/dP) (own rows), both updated in place to the values before the
// token.  With S = sym(dL/dP_new) and dL/dM_new including q gy^T:
//   ge = beta gM^T u (= dL/dv),  a = gM e,  w = S u,  z = u.(a - w)
//   gs = (s > floor) ? -z beta^2 : 0 (= dL/dr)
//   gu = beta (a - 2 w) + gs k
//   dL/dk = -(d*M_prev) ge + gs u + P' gu,   dL/dq = M_new gy
//   H = S + sym(gu k^T),  dL/dd_i = 2 sum_j H_ij d_j P_ij + sum_c (gM - k ge^T)_ic M_ic
//   dL/dp = trace(H),  S_prev = H * d d^T,  gM_prev = (gM - k ge^T) * d
// At the first token the full (asymmetric) adjoint of the initial covariance
// (S + gu k^T) * d d^T is stored in gc0r.  DYN = false skips dL/dd and dL/dp
// and reports zeros for dd/dp/dr (the fixed-dynamics ABI returns zeros).
template <int D, int M, int G, bool DYN>
__device__ __forceinline__ void reverse_step(const TokenIn<D, M, G>& in, const RevIn<D, M, G>& x,
                                             ColsArr<D, M, G>& gM,
                                             RowsArr<D, M, G>& Gs,
                                             const RowsArr<D, M, G>& eye, float floor, int g,
                                             int lane, bool first_token,
                                             RowsArr<D, M, G>& gc0r, RevOut<D, M, G>& o) {
  using L = Layout<D, M, G>;
  constexpr int RPL = L::RPL, CPL = L::CPL;
  const bool writer = L::row_writer(g);
  const float beta = x.beta;

  // Value-column part: own columns, partial row sums for the group.
  float gqp[D], ap[D], gkp[D], gdp[D];
#pragma unroll
  for (int i = 0; i < D; ++i) gqp[i] = ap[i] = gkp[i] = gdp[i] = 0.f;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const float bu = beta * x.u[i];
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) {
      gqp[i] = fmaf(fmaf(bu, x.e[cc], x.mp[i][cc]), x.gy[cc], gqp[i]);
      gM[i][cc] = fmaf(x.q[i], x.gy[cc], gM[i][cc]);
    }
  }
  float ge[CPL];
#pragma unroll
  for (int cc = 0; cc < CPL; ++cc) {
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < D; ++i) z = fmaf(gM[i][cc], x.u[i], z);
    ge[cc] = beta * z;
    o.gv[cc] = ge[cc];
  }
#pragma unroll
  for (int i = 0; i < D; ++i) {
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) {
      ap[i] = fmaf(gM[i][cc], x.e[cc], ap[i]);
      gkp[i] = fmaf(-x.mp[i][cc], ge[cc], gkp[i]);
      const float gmb = fmaf(-in.k[i], ge[cc], gM[i][cc]);
      if constexpr (DYN) gdp[i] = fmaf(gmb, x.Mprev[i][cc], gdp[i]);
      gM[i][cc] = gmb * in.d[i];
    }
  }
  float a_own[RPL], gkc[RPL], gdc[RPL];
  group_reduce_rows<D, G>(ap, a_own, g);
  group_reduce_rows<D, G>(gkp, gkc, g);
  group_reduce_rows<D, G>(gqp, o.gq_own, g);
  if constexpr (DYN) group_reduce_rows<D, G>(gdp, gdc, g);

  // Covariance-row part.
  float w_own[RPL];
  float zp = 0.f;
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj) {
    float w = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) w = fmaf(Gs[jj][j], x.u[j], w);
    w_own[jj] = w;
    zp = fmaf(x.u_own[jj], a_own[jj] - w, zp);
  }
  const float z = group_sum<G>(writer ? zp : 0.f);
  const float gs = (x.s > floor) ? -z * beta * beta : 0.f;
  float gu_own[RPL], gu[D];
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj) gu_own[jj] = fmaf(beta, a_own[jj] - 2.f * w_own[jj], gs * in.k_own[jj]);
  gather_rows<D, M, G>(gu_own, gu, lane);

  float gpp = 0.f;
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj) {
    float gk = fmaf(gs, x.u_own[jj], gkc[jj]);
    float gd = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const float dd = in.d_own[jj] * in.d[j];
      gk = fmaf(x.Pb[jj][j], gu[j], gk);
      const float hsym = fmaf(0.5f, gu_own[jj] * in.k[j] + gu[j] * in.k_own[jj], Gs[jj][j]);
      if constexpr (DYN) {
        gd = fmaf(hsym * in.d[j], x.Pprev[jj][j], gd);
        gpp = fmaf(hsym, eye[jj][j], gpp);
      }
      if (first_token) gc0r[jj][j] = fmaf(gu_own[jj], in.k[j], Gs[jj][j]) * dd;
      Gs[jj][j] = hsym * dd;
    }
    o.gk_own[jj] = gk;
    o.gd_own[jj] = DYN ? fmaf(2.f, gd, gdc[jj]) : 0.f;
  }
  o.gp = DYN ? group_sum<G>(writer ? gpp : 0.f) : 0.f;
  o.gr = DYN ? gs : 0.f;
}

// sin and cos of x without a library call (an outlined call makes the
// caller save its live registers to scratch).  Cody-Waite reduction by pi/2
// in double precision (pi/2 as a two-double sum; n x pi/2 is exact in the
// fma for any |x| below 2^40), then the Taylor series on |r| <= pi/4:
// sin to r^9 (next term below 7e-10 relative) and cos to r^10 (below 1.2e-10).
__device__ __forceinline__ void sincos_rad(float x, float& s, float& c) {
  const double xd = x;
  const double n = rint(xd * 0.6366197723675814);
  const double rd = fma(-n, 6.123233995736766e-17, fma(-n, 1.5707963267948966, xd));
  const float r = static_cast<float>(rd), r2 = r * r;
  float ps = 1.f / 362880.f;
  ps = fmaf(ps, r2, -1.f / 5040.f);
  ps = fmaf(ps, r2, 1.f / 120.f);
  ps = fmaf(ps, r2, -1.f / 6.f);
  const float sr = fmaf(r * r2, ps, r);
  float pc = -1.f / 3628800.f;
  pc = fmaf(pc, r2, 1.f / 40320.f);
  pc = fmaf(pc, r2, -1.f / 720.f);
  pc = fmaf(pc, r2, 1.f / 24.f);
  pc = fmaf(pc, r2, -0.5f);
  const float cr = fmaf(r2, pc, 1.f);
  const int q = static_cast<int>(static_cast<int64_t>(n) & 3);
  s = (q == 0) ? sr : (q == 1) ? cr : (q == 2) ? -sr : -cr;
  c = (q == 0) ? cr : (q == 1) ? -sr : (q == 2) ? -cr : sr;
}

}  // namespace bssm
