// gfx950 kernels for the exact dense-covariance recurrence with
// block-diagonal damped 2-D rotations (bayes_ssm/bayesian_layer.py:254-323).
//
// Pair k = state rows (2k, 2k+1) turns by R_k = [[c, -s], [s, c]] with
// c = rho cos(theta), s = rho sin(theta), rho = min(max(radius, tiny), 1),
// and its process variance is added to entry (2k, 2k) only:
//   P' = R P R^T + Q     M' = R M     u = P' k     s = r + k.u
//   beta = 1 / max(s, floor)          e = v - M'^T k
//   M <- M' + beta u e^T              P <- P' - beta u u^T      y = M^T q
// (the reference symmetrises P after every token; here P' is formed in a
// symmetric summation order, so P stays bitwise symmetric as in the
// diagonal kernels).
//
// Work decomposition as the diagonal kernels (bssm_common.h): a group of G
// lanes per sequence, covariance rows round-robin over the group, value
// columns split.  The two rows of a pair always sit in lanes g and g ^ 1 at
// the same slot, so the row mixing of R is one DPP exchange; the column
// mixing is local.  P'_ij sums its four terms t_ab = (R_ia R_jb) P_ab as
// (t00 + t11) + (t01 + t10), which the owners of rows i and j evaluate to the
// same bits.
//
// The backward replays each checkpoint chunk on chip and reverses it.  Per
// token, with H = S + sym(gu k^T) (S = sym(dL/dP_new)) the adjoint of P':
//   S_prev = R^T H R,   gM_prev = R^T (gM - k ge^T),
//   dL/dR = 2 H R P_prev + (gM - k ge^T) M_prev^T  (pair blocks only),
//   dL/dc_k = dR_{2k,2k} + dR_{2k+1,2k+1},  dL/ds_k = dR_{2k+1,2k} - dR_{2k,2k+1},
//   dL/dtheta = rho (dL/ds cos - dL/dc sin),  dL/drho = dL/dc cos + dL/ds sin
//   (zero where the radius clamp is active), dL/dq_k = H_{2k,2k}.
// The initial-covariance adjoint keeps the asymmetric convention of the
// diagonal kernels: R^T (S + gu k^T) R at the first token.

#include <cfloat>

#include "bssm_rot4.h"
#include "bssm_step.h"

// No contraction (except in the reverse arithmetic of the backward): the
// four-term sums of P' would otherwise be fused as fma(first product,
// second), which the owners of rows i and j evaluate with the products in
// swapped roles, so P_ij and P_ji would differ in the last bit.  Every
// intended fused multiply-add is an explicit fmaf.
#pragma clang fp contract(off)

namespace bssm {
namespace rot {
namespace {

constexpr float kTiny = FLT_MIN;  // torch.finfo(float32).tiny

template <int D, int M, int G>
struct TokRot {
  using L = Layout<D, M, G>;
  static constexpr int J = D / 2;
  float k[D], k_own[L::RPL];
  float v[L::CPL];
  float c[J], sn[J];    // rotation coefficients of every pair
  float cs[J], si[J];   // cos, sin of the angles (backward)
  float rho[J];         // clamped radii
  bool live[J];         // the radius clamp passes gradients
  float p[J], r;
};

// Rotation-dynamics tile pointers of one sequence (cs, si: cos and sin of
// the staged angles, filled by fill_trig; cs is the angle tile itself).
struct RotTile {
  const float* k;
  const float* v;
  const float* rad;
  const float* ang;
  const float* p;
  const float* r;
  const float* cs;
  const float* si;
};

// cos and sin of every angle of a staged tile (SPW sequence rows of TTT
// tokens x J pairs in the padded Tile<J, TTT> layout), each computed once per
// wave: every lane of a sequence's group reads them instead of evaluating
// sincos_rad for every pair itself.  cos replaces the angle in place (the
// kernels need only the two values), sin goes to si.
template <int SPW, int J, int TTT>
__device__ __forceinline__ void fill_trig(float* ang, float* si, int lane) {
  constexpr int PER = TTT * J, STRIDE = Tile<J, TTT>::STRIDE, TOTAL = SPW * PER;
#pragma unroll
  for (int it = 0; it < (TOTAL + kWave - 1) / kWave; ++it) {
    const int f = it * kWave + lane;
    if (f < TOTAL) {
      const int idx = (f / PER) * STRIDE + f % PER;
      float sa, ca;
      sincos_rad(ang[idx], sa, ca);
      ang[idx] = ca;
      si[idx] = sa;
    }
  }
}

template <int D, int M, int G>
__device__ __forceinline__ void read_rot(TokRot<D, M, G>& in, const RotTile& st, int tt, int g, bool need_v) {
  using L = Layout<D, M, G>;
  constexpr int J = D / 2;
#pragma unroll
  for (int j = 0; j < D; ++j) in.k[j] = st.k[tt * D + j];
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj) in.k_own[jj] = st.k[tt * D + L::row(g, jj)];
#pragma unroll
  for (int m = 0; m < J; ++m) {
    const float rc = fmaxf(st.rad[tt * J + m], kTiny);
    in.live[m] = st.rad[tt * J + m] >= kTiny && rc <= 1.f;
    in.rho[m] = rc <= 1.f ? rc : 1.f;
    const float ca = st.cs[tt * J + m], sa = st.si[tt * J + m];
    in.cs[m] = ca;
    in.si[m] = sa;
    in.c[m] = in.rho[m] * ca;
    in.sn[m] = in.rho[m] * sa;
    in.p[m] = st.p[tt * J + m];
  }
  in.r = st.r[tt];
  if (need_v) {
#pragma unroll
    for (int c = 0; c < L::CPL; ++c) in.v[c] = st.v[tt * M + g * L::CPL + c];
  }
}

// Element k of a small register array for a lane-dependent k, by selects
// (indexing with it would move the array to scratch memory).  The empty asm
// makes each element an opaque register value, so the selects are not
// folded back into one indexed load.
template <int J>
__device__ __forceinline__ float pick(const float (&x)[J], int k) {
  uint32_t v = __builtin_bit_cast(uint32_t, x[0]);
#pragma unroll
  for (int m = 1; m < J; ++m) {
    const uint32_t mask = 0u - static_cast<uint32_t>(k == m);
    v = (__builtin_bit_cast(uint32_t, x[m]) & mask) | (v & ~mask);
  }
  return __builtin_bit_cast(float, v);
}

// R_{i, a} for a = 2 (i >> 1) + t (t = 0, 1), and the transposed R_{a, i}.
template <int J>
__device__ __forceinline__ float r_row(const float (&c)[J], const float (&s)[J], int i, int t) {
  const int k = i >> 1;
  const float ck = pick<J>(c, k), sk = pick<J>(s, k);
  if (i & 1) return t ? ck : sk;
  return t ? -sk : ck;
}
template <int J>
__device__ __forceinline__ float r_col(const float (&c)[J], const float (&s)[J], int i, int t) {
  const int k = i >> 1;
  const float ck = pick<J>(c, k), sk = pick<J>(s, k);
  if (i & 1) return t ? ck : -sk;
  return t ? sk : ck;
}

// X_ij = sum_{a in pair(i), b in pair(j)} A_ia X0_ab A_jb for the lane's own
// rows, A = R (TRANS false) or R^T (TRANS true).  own[jj] is row(g, jj) of
// X0, part[jj] the partner row (row ^ 1).  Each term is (A_ia A_jb) X0_ab,
// summed as ((own, b0) + (part, b1)) + ((own, b1) + (part, b0)): for an even
// row that is (t00 + t11) + (t01 + t10) in pair positions, for an odd row
// (t10 + t01) + (t11 + t00), so the owners of rows i and j evaluate X_ij and
// X_ji to the same bits, and no lane-dependent operand selection is needed.
// Coefficients: A_{i,own} = c, A_{i,part} = -s (R, even i), s (R, odd i),
// s (R^T, even i), -s (R^T, odd i); for the columns of pair m,
//   R:   A_{2m,b} = (c, -s), A_{2m+1,b} = (s, c);
//   R^T: A_{2m,b} = (c, s),  A_{2m+1,b} = (-s, c);
// the four coefficient products of a column pair are formed once.
template <int D, int M, int G, bool TRANS>
__device__ __forceinline__ void sandwich(const float (&c)[D / 2], const float (&s)[D / 2], const RowsArr<D, M, G>& own,
                                         const RowsArr<D, M, G>& part, int g, RowsArr<D, M, G>& out) {
  using L = Layout<D, M, G>;
  constexpr int J = D / 2;
  constexpr float sg = TRANS ? 1.f : -1.f;
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj) {
    const int i = L::row(g, jj);
    const float ao = pick<J>(c, i >> 1), sk = pick<J>(s, i >> 1);
    const float ap = ((i & 1) != 0) != TRANS ? sk : -sk;
#pragma unroll
    for (int m = 0; m < J; ++m) {
      const float oc = ao * c[m], os = ao * s[m], pc = ap * c[m], ps = ap * s[m];
      const float xo0 = own[jj][2 * m], xo1 = own[jj][2 * m + 1];
      const float xp0 = part[jj][2 * m], xp1 = part[jj][2 * m + 1];
      out[jj][2 * m] = (oc * xo0 + (sg * ps) * xp1) + ((sg * os) * xo1 + pc * xp0);
      out[jj][2 * m + 1] = ((-sg * os) * xo0 + pc * xp1) + (oc * xo1 + (-sg * ps) * xp0);
    }
  }
}

template <int D, int M, int G>
__device__ __forceinline__ void partner_rows(const RowsArr<D, M, G>& x, RowsArr<D, M, G>& y) {
  using L = Layout<D, M, G>;
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj)
#pragma unroll
    for (int j = 0; j < D; ++j) y[jj][j] = xor_lane<0>(x[jj][j]);
}

// One forward token.  Pb receives P' (own rows).
template <int D, int M, int G>
__device__ __forceinline__ void step_rot(Belief<D, M, G>& b, const TokRot<D, M, G>& in, float floor, int g, int lane,
                                         StepOut<D, M, G>& o, RowsArr<D, M, G>& Pb) {
  using L = Layout<D, M, G>;
  constexpr int J = D / 2;
  float Pn[L::RPL][D];
  partner_rows<D, M, G>(b.P, Pn);
  sandwich<D, M, G, false>(in.c, in.sn, b.P, Pn, g, Pb);
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj) {
    const int i = L::row(g, jj);
    if (!(i & 1)) {
#pragma unroll
      for (int j = 0; j < D; j += 2)
        if (j == i) Pb[jj][j] += in.p[j >> 1];
    }
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) acc = fmaf(Pb[jj][j], in.k[j], acc);
    o.u_own[jj] = acc;
  }
  gather_rows<D, M, G>(o.u_own, o.u, lane);
  float s = in.r;
#pragma unroll
  for (int j = 0; j < D; ++j) s = fmaf(in.k[j], o.u[j], s);
  o.s = s;
  const float beta = fast_rcp(fmaxf(s, floor));
#pragma unroll
  for (int cc = 0; cc < L::CPL; ++cc) {
    float mr[D];
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int a0 = i & ~1;
      mr[i] = fmaf(r_row<J>(in.c, in.sn, i, 1), b.Mv[a0 + 1][cc], r_row<J>(in.c, in.sn, i, 0) * b.Mv[a0][cc]);
    }
    float e = in.v[cc];
#pragma unroll
    for (int i = 0; i < D; ++i) e = fmaf(-mr[i], in.k[i], e);
    o.e[cc] = e;
#pragma unroll
    for (int i = 0; i < D; ++i) b.Mv[i][cc] = fmaf(beta * o.u[i], e, mr[i]);
  }
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj)
#pragma unroll
    for (int j = 0; j < D; ++j) b.P[jj][j] = fmaf(-beta, o.u_own[jj] * o.u[j], Pb[jj][j]);
}

template <int D, int M, int G>
struct RotHist {
  using L = Layout<D, M, G>;
  float Pp[L::RPL][D];  // covariance rows before the token
  float Mp[D][L::CPL];  // mean block before the token
  float u[D];
  float u_own[L::RPL];
  float s;
  float e[L::CPL];
};

template <int D, int M, int G>
struct RotOut {
  using L = Layout<D, M, G>;
  float gk_own[L::RPL], gq_own[L::RPL];
  float gv[L::CPL];
  float grad_rad[D / 2], grad_ang[D / 2], gp[D / 2];
  float gr;
};

// Reverse of one token (see the header comment).  gM, Gs: carried adjoints,
// updated in place.
template <int D, int M, int G>
__device__ __forceinline__ void reverse_rot(const TokRot<D, M, G>& in, const RotHist<D, M, G>& h,
                                            const float (&q)[D], const float (&gy)[Layout<D, M, G>::CPL],
                                            ColsArr<D, M, G>& gM, RowsArr<D, M, G>& Gs, float floor, int g,
                                            int lane, bool first_token, RowsArr<D, M, G>& gc0r,
                                            RotOut<D, M, G>& o) {
  // The adjoint arithmetic may contract (the replayed P' comes from
  // sandwich / step_rot, which do not, so it is bitwise the forward's).
#pragma clang fp contract(fast)
  using L = Layout<D, M, G>;
  constexpr int RPL = L::RPL, CPL = L::CPL, J = D / 2;
  const bool writer = L::row_writer(g);
  const float beta = fast_rcp(fmaxf(h.s, floor));

  // P' (own rows) and M' = R M_prev (own columns), recomputed from the history.
  float Pb[RPL][D];
  {
    float Pn[RPL][D];
    partner_rows<D, M, G>(h.Pp, Pn);
    sandwich<D, M, G, false>(in.c, in.sn, h.Pp, Pn, g, Pb);
#pragma unroll
    for (int jj = 0; jj < RPL; ++jj) {
      const int i = L::row(g, jj);
#pragma unroll
      for (int j = 0; j < D; j += 2)
        if (j == i) Pb[jj][j] += in.p[j >> 1];
    }
  }
  float mp[D][CPL];
#pragma unroll
  for (int cc = 0; cc < CPL; ++cc)
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int a0 = i & ~1;
      mp[i][cc] = fmaf(r_row<J>(in.c, in.sn, i, 1), h.Mp[a0 + 1][cc], r_row<J>(in.c, in.sn, i, 0) * h.Mp[a0][cc]);
    }

  // Value-column part.
  float gqp[D], ap[D], gkp[D];
#pragma unroll
  for (int i = 0; i < D; ++i) gqp[i] = ap[i] = gkp[i] = 0.f;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const float bu = beta * h.u[i];
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) {
      gqp[i] = fmaf(fmaf(bu, h.e[cc], mp[i][cc]), gy[cc], gqp[i]);
      gM[i][cc] = fmaf(q[i], gy[cc], gM[i][cc]);
    }
  }
  float ge[CPL];
#pragma unroll
  for (int cc = 0; cc < CPL; ++cc) {
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < D; ++i) z = fmaf(gM[i][cc], h.u[i], z);
    ge[cc] = beta * z;
    o.gv[cc] = ge[cc];
  }
  float gcm[J], gsm[J];
#pragma unroll
  for (int m = 0; m < J; ++m) gcm[m] = gsm[m] = 0.f;
#pragma unroll
  for (int cc = 0; cc < CPL; ++cc) {
    float gmb[D];
#pragma unroll
    for (int i = 0; i < D; ++i) {
      ap[i] = fmaf(gM[i][cc], h.e[cc], ap[i]);
      gkp[i] = fmaf(-mp[i][cc], ge[cc], gkp[i]);
      gmb[i] = fmaf(-in.k[i], ge[cc], gM[i][cc]);
    }
#pragma unroll
    for (int m = 0; m < J; ++m) {
      const float g0 = gmb[2 * m], g1 = gmb[2 * m + 1];
      const float m0 = h.Mp[2 * m][cc], m1 = h.Mp[2 * m + 1][cc];
      gcm[m] = fmaf(g0, m0, fmaf(g1, m1, gcm[m]));
      gsm[m] = fmaf(g1, m0, fmaf(-g0, m1, gsm[m]));
      gM[2 * m][cc] = fmaf(in.sn[m], g1, in.c[m] * g0);
      gM[2 * m + 1][cc] = fmaf(-in.sn[m], g0, in.c[m] * g1);
    }
  }
#pragma unroll
  for (int m = 0; m < J; ++m) {
    gcm[m] = group_sum<G>(gcm[m]);
    gsm[m] = group_sum<G>(gsm[m]);
  }
  float a_own[RPL], gkc[RPL];
  group_reduce_rows<D, G>(ap, a_own, g);
  group_reduce_rows<D, G>(gkp, gkc, g);
  group_reduce_rows<D, G>(gqp, o.gq_own, g);

  // Covariance-row part.
  float w_own[RPL];
  float zp = 0.f;
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj) {
    float w = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) w = fmaf(Gs[jj][j], h.u[j], w);
    w_own[jj] = w;
    zp = fmaf(h.u_own[jj], a_own[jj] - w, zp);
  }
  const float z = group_sum<G>(writer ? zp : 0.f);
  // The reference runs this core in torch, where clamp_min passes the
  // gradient at s == floor too (the diagonal kernels' gate is strict).
  const float gs = (h.s >= floor) ? -z * beta * beta : 0.f;
  float gu_own[RPL], gu[D];
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj) gu_own[jj] = fmaf(beta, a_own[jj] - 2.f * w_own[jj], gs * in.k_own[jj]);
  gather_rows<D, M, G>(gu_own, gu, lane);

  float H[RPL][D];
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj) {
    float gk = fmaf(gs, h.u_own[jj], gkc[jj]);
#pragma unroll
    for (int j = 0; j < D; ++j) {
      gk = fmaf(Pb[jj][j], gu[j], gk);
      H[jj][j] = fmaf(0.5f, gu_own[jj] * in.k[j] + gu[j] * in.k_own[jj], Gs[jj][j]);
    }
    o.gk_own[jj] = gk;
  }

  // dL/dR from the covariance: 2 H R P_prev on the pair blocks.  Y = P_prev R^T
  // (row a of it is row a of P_prev with its columns mixed by R).
  float Y[RPL][D], Yn[RPL][D];
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int b0 = j & ~1;
      Y[jj][j] = fmaf(r_row<J>(in.c, in.sn, j, 1), h.Pp[jj][b0 + 1], r_row<J>(in.c, in.sn, j, 0) * h.Pp[jj][b0]);
    }
  partner_rows<D, M, G>(Y, Yn);
  float gcp[J], gsp[J], gpp[J];
#pragma unroll
  for (int m = 0; m < J; ++m) gcp[m] = gsp[m] = gpp[m] = 0.f;
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj) {
    const int i = L::row(g, jj);
    float self = 0.f, cross = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      self = fmaf(H[jj][j], Y[jj][j], self);
      cross = fmaf(H[jj][j], Yn[jj][j], cross);
    }
    // Row i even: dR_{i,i} = 2 self, dR_{i,i+1} = 2 cross; odd: dR_{i,i} = 2 self, dR_{i,i-1} = 2 cross.
    const int m = i >> 1;
    float hii = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) hii = (j == i) ? H[jj][j] : hii;
#pragma unroll
    for (int mm = 0; mm < J; ++mm) {
      if (mm == m) {
        gcp[mm] += 2.f * self;
        gsp[mm] += (i & 1) ? 2.f * cross : -2.f * cross;
        if (!(i & 1)) gpp[mm] += hii;
      }
    }
  }
  // The two rows of a pair are in lanes g and g ^ 1; with replicated rows
  // (D < G) each lane pair holds a full copy.
#pragma unroll
  for (int m = 0; m < J; ++m) {
    float cp = gcp[m], sp = gsp[m], pq = gpp[m];
    if constexpr (D >= G) {
      // Rows of pair m: lanes owner(2m), owner(2m) + 1; other lanes hold 0.
      cp = group_sum<G>(cp);
      sp = group_sum<G>(sp);
      pq = group_sum<G>(pq);
    } else {
      cp += xor_lane<0>(cp);
      sp += xor_lane<0>(sp);
      pq += xor_lane<0>(pq);
    }
    const float gc = gcm[m] + cp, gsn = gsm[m] + sp;
    o.grad_rad[m] = in.live[m] ? fmaf(gc, in.cs[m], gsn * in.si[m]) : 0.f;
    o.grad_ang[m] = in.rho[m] * fmaf(gsn, in.cs[m], -gc * in.si[m]);
    o.gp[m] = pq;
  }
  o.gr = gs;

  // Carried covariance adjoint S_prev = R^T H R (and the asymmetric initial
  // adjoint R^T (S + gu k^T) R at the first token).
  {
    float Hn[RPL][D];
    partner_rows<D, M, G>(H, Hn);
    if (first_token) {
      float A[RPL][D], An[RPL][D];
#pragma unroll
      for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
        for (int j = 0; j < D; ++j) A[jj][j] = fmaf(gu_own[jj], in.k[j], Gs[jj][j]);
      partner_rows<D, M, G>(A, An);
      sandwich<D, M, G, true>(in.c, in.sn, A, An, g, gc0r);
    }
    sandwich<D, M, G, true>(in.c, in.sn, H, Hn, g, Gs);
  }
}

// ------------------------------------------------------------------ kernels
template <int D, int M, int G, int TT>
__global__ __launch_bounds__(kWave) void forward_kernel(RotArgs a) {
  using L = Layout<D, M, G>;
  constexpr int SPW = L::SPW, J = D / 2;
  constexpr int SD = Tile<D, TT>::STRIDE, SM = Tile<M, TT>::STRIDE, SJ = Tile<J, TT>::STRIDE,
                S1 = Tile<1, TT>::STRIDE;
  __shared__ float sk[SPW * SD];
  __shared__ float sq[SPW * SD];
  __shared__ float sv[SPW * SM];  // values in, readouts out
  __shared__ float srad[SPW * SJ];
  __shared__ float sang[SPW * SJ];
  __shared__ float sp[SPW * SJ];
  __shared__ float sr[SPW * S1];
  __shared__ float ssi[SPW * SJ];

  const int lane = threadIdx.x;
  const int g = lane % G;
  const int s = lane / G;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t n = n0 + s;
  const bool active = n < a.n;
  const int64_t na = active ? n : 0;
  const int64_t T = a.t;

  Belief<D, M, G> b;
  load_belief<D, M, G>(b, a.m0 + na * D * M, a.c0 + na * D * D, g, active);
  // The initial belief has landed before the token loop: otherwise the
  // compiler's wait bookkeeping keeps its loads pending at the loop header
  // and waits for every outstanding load (the next tile's prefetch too) at
  // the belief's first use in each iteration.
  r4::vm_wait<0>();
  const int64_t bm_seq = (a.nb + 1) * D * M, bc_seq = (a.nb + 1) * D * D;
  if (active) store_belief<D, M, G>(b, a.bm + na * bm_seq, a.bc + na * bc_seq, g);

  RotTile st{sk + s * SD, sv + s * SM, srad + s * SJ, sang + s * SJ, sp + s * SJ, sr + s * S1, sang + s * SJ,
             ssi + s * SJ};
  const float* qs = sq + s * SD;
  float* ys = sv + s * SM;
  // With every stream 16-byte aligned the next tile is loaded into
  // registers while this one is computed; otherwise tiles are staged
  // synchronously.
  TileRegs<D, TT, SPW> rk, rq;
  TileRegs<M, TT, SPW> rv;
  TileRegs<J, TT, SPW> rrad, rang, rp;
  TileRegs<1, TT, SPW> rr;
  auto issue = [&](int64_t t0) {
    const int len = tile_len(T, t0, TT);
    rk.load(a.k, n0, a.n, T, t0, len, lane);
    rq.load(a.q, n0, a.n, T, t0, len, lane);
    rv.load(a.v, n0, a.n, T, t0, len, lane);
    rrad.load(a.rad, n0, a.n, T, t0, len, lane);
    rang.load(a.ang, n0, a.n, T, t0, len, lane);
    rp.load(a.p, n0, a.n, T, t0, len, lane);
    rr.load(a.r, n0, a.n, T, t0, len, lane);
  };
  if (a.vec && T > 0) issue(0);
  int64_t next_ckpt = a.chunk, ckpt = 1;
  // Eight tokens of a staged tile, unrolled: each token's LDS reads are
  // issued before the previous token is computed (the scheduling barriers
  // keep them there), so a token does not wait out the LDS latency.
  struct FwdIn {
    TokRot<D, M, G> t;
    float q[D];
  };
  auto read_in = [&](FwdIn& x, int tt) __attribute__((always_inline)) {
    read_rot<D, M, G>(x.t, st, tt, g, true);
#pragma unroll
    for (int i = 0; i < D; ++i) x.q[i] = qs[tt * D + i];
  };
  auto step_y = [&](const FwdIn& x, int tt) __attribute__((always_inline)) {
    StepOut<D, M, G> o;
    float Pb[L::RPL][D];
    step_rot<D, M, G>(b, x.t, a.floor, g, lane, o, Pb);
#pragma unroll
    for (int c = 0; c < L::CPL; ++c) {
      float y = 0.f;
#pragma unroll
      for (int i = 0; i < D; ++i) y = fmaf(b.Mv[i][c], x.q[i], y);
      ys[tt * M + g * L::CPL + c] = y;
    }
  };
  auto run8 = [&](int base) __attribute__((always_inline)) {
    FwdIn x[8];
    read_in(x[0], base);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i + 1 < 8) read_in(x[i + 1], base + i + 1);
      __builtin_amdgcn_sched_barrier(0);
      step_y(x[i], base + i);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int64_t t0 = 0; t0 < T; t0 += TT) {
    const int len = tile_len(T, t0, TT);
    if (a.vec) {
      rk.commit(sk, lane);
      rq.commit(sq, lane);
      rv.commit(sv, lane);
      rrad.commit(srad, lane);
      rang.commit(sang, lane);
      rp.commit(sp, lane);
      rr.commit(sr, lane);
    } else {
      stage_in<D, TT, SPW>(sk, a.k, n0, a.n, T, t0, len, false, lane);
      stage_in<D, TT, SPW>(sq, a.q, n0, a.n, T, t0, len, false, lane);
      stage_in<M, TT, SPW>(sv, a.v, n0, a.n, T, t0, len, false, lane);
      stage_in<J, TT, SPW>(srad, a.rad, n0, a.n, T, t0, len, false, lane);
      stage_in<J, TT, SPW>(sang, a.ang, n0, a.n, T, t0, len, false, lane);
      stage_in<J, TT, SPW>(sp, a.p, n0, a.n, T, t0, len, false, lane);
      stage_in<1, TT, SPW>(sr, a.r, n0, a.n, T, t0, len, false, lane);
    }
    __syncthreads();
    fill_trig<SPW, J, TT>(sang, ssi, lane);
    __syncthreads();
    if (a.vec && t0 + TT < T) issue(t0 + TT);
    if (len == TT && TT % 8 == 0 && a.chunk % 8 == 0) {
      // Whole tile, checkpoints on 8-token boundaries only.
#pragma unroll
      for (int h = 0; h < TT / 8; ++h) {
        if (t0 + 8 * h == next_ckpt) {
          if (active)
            store_belief<D, M, G>(b, a.bm + na * bm_seq + ckpt * D * M, a.bc + na * bc_seq + ckpt * D * D, g);
          ++ckpt;
          next_ckpt += a.chunk;
        }
        run8(8 * h);
      }
    } else {
      for (int tt = 0; tt < len; ++tt) {
        if (t0 + tt == next_ckpt) {
          if (active)
            store_belief<D, M, G>(b, a.bm + na * bm_seq + ckpt * D * M, a.bc + na * bc_seq + ckpt * D * D, g);
          ++ckpt;
          next_ckpt += a.chunk;
        }
        FwdIn x;
        read_in(x, tt);
        step_y(x, tt);
      }
    }
    __syncthreads();
    stage_out<M, TT, SPW>(sv, a.y, n0, a.n, T, t0, len, a.vec, lane);
    __syncthreads();
  }
  if (active) {
    store_belief<D, M, G>(b, a.mT + na * D * M, a.cT + na * D * D, g);
    if (T > 0) store_belief<D, M, G>(b, a.bm + na * bm_seq + a.nb * D * M, a.bc + na * bc_seq + a.nb * D * D, g);
  }
}

// LDS-DMA staging of one checkpoint chunk for the backward: each
// stream's rows of the wave's SPW sequences land unpadded, [seq][R floats],
// in a region rounded up to whole 1 KB instructions (lanes past the last
// sequence load nothing and fill the region's tail with zeros).
constexpr int stage_region(int spw, int r) { return (spw * r + 255) / 256 * 256; }

// Rows of R floats per sequence from global rows `row` bytes apart, starting
// `base` bytes into each row; W > 0: a token stream of W floats per token
// (pieces whose first token is at or past T are skipped), W = 0: records.
template <int SPW, int R, int W>
__device__ __forceinline__ void dma_rows(r4::Rsrc rs, float* dst, uint32_t row, uint32_t base, uint32_t ts,
                                         uint32_t T, int lane) {
  constexpr int NI = (SPW * R + 255) / 256;
  constexpr bool kNt = R * 4 >= 128;  // nontemporal where a row piece covers whole 128-byte lines
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const uint32_t f = 256u * i + 4u * lane;
    const uint32_t sq = f / R, o = f % R;
    const bool ok = sq < static_cast<uint32_t>(SPW) && (W == 0 || ts + o / (W > 0 ? W : 1) < T);
    r4::dma16<kNt>(rs, dst + 256 * i, ok ? sq * row + base + 4u * o : r4::kOob);
  }
}

// Unpadded staged rows into the padded tile layout the kernels read.
template <int SPW, int W, int SUB>
__device__ __forceinline__ void copy_rows(const float* src, float* dst, int lane) {
  constexpr int R = SUB * W, TOTAL = SPW * R;
#pragma unroll
  for (int it = 0; it < (TOTAL + 255) / 256; ++it) {
    const int f = 256 * it + 4 * lane;
    if (f < TOTAL) {
      const int sq = f / R, o = f % R;
      *reinterpret_cast<v4f*>(dst + sq * Tile<W, SUB>::STRIDE + o) = *reinterpret_cast<const v4f*>(src + f);
    }
  }
}

template <int D, int M, int G, int SUB>
__global__ __launch_bounds__(kWave) void backward_kernel(RotArgs a) {
#pragma clang fp contract(fast)
  using L = Layout<D, M, G>;
  constexpr int SPW = L::SPW, RPL = L::RPL, CPL = L::CPL, J = D / 2;
  constexpr int SD = Tile<D, SUB>::STRIDE, SM = Tile<M, SUB>::STRIDE, SJ = Tile<J, SUB>::STRIDE,
                S1 = Tile<1, SUB>::STRIDE;
  // Input tiles are overwritten in place by their gradients; sg holds gy.
  __shared__ float sk[SPW * SD];
  __shared__ float sq[SPW * SD];
  __shared__ float sv[SPW * SM];
  __shared__ float sg[SPW * SM];
  __shared__ float srad[SPW * SJ];
  __shared__ float sang[SPW * SJ];
  __shared__ float sp[SPW * SJ];
  __shared__ float sr[SPW * S1];
  __shared__ float ssi[SPW * SJ];
  // LDS-DMA staging of the next chunk (see dma_rows).
  constexpr int RK = stage_region(SPW, SUB * D), RV = stage_region(SPW, SUB * M), RJ = stage_region(SPW, SUB * J),
                R1 = stage_region(SPW, SUB), RBM = stage_region(SPW, D * M), RBC = stage_region(SPW, D * D);
  constexpr int OK = 0, OQ = RK, OV = 2 * RK, OG = OV + RV, ORAD = OG + RV, OANG = ORAD + RJ, OP = OANG + RJ,
                OR = OP + RJ, OBM = OR + R1, OBC = OBM + RBM, STG = OBC + RBC;
  __shared__ float stg[STG];

  const int lane = threadIdx.x;
  const int g = lane % G;
  const int s = lane / G;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t n = n0 + s;
  const bool active = n < a.n;
  const int64_t na = active ? n : 0;
  const int64_t T = a.t;
  const bool writer = L::row_writer(g);

  float gM[D][CPL];
  float Gs[RPL][D];
#pragma unroll
  for (int i = 0; i < D; ++i)
#pragma unroll
    for (int c = 0; c < CPL; ++c) gM[i][c] = (active && a.gmf) ? a.gmf[na * D * M + i * M + g * CPL + c] : 0.f;
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj) {
    const int rr = L::row(g, jj);
#pragma unroll
    for (int j = 0; j < D; ++j)
      Gs[jj][j] = (active && a.gcf) ? 0.5f * (a.gcf[na * D * D + rr * D + j] + a.gcf[na * D * D + j * D + rr]) : 0.f;
  }
  float gc0r[RPL][D];
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
    for (int j = 0; j < D; ++j) gc0r[jj][j] = 0.f;

  RotTile st{sk + s * SD, sv + s * SM, srad + s * SJ, sang + s * SJ, sp + s * SJ, sr + s * S1, sang + s * SJ,
             ssi + s * SJ};
  float* gks = sk + s * SD;
  float* gqs = sq + s * SD;
  float* gvs = sv + s * SM;
  const float* gys = sg + s * SM;
  float* grads = srad + s * SJ;
  float* gangs = sang + s * SJ;
  float* gps = sp + s * SJ;
  float* grs = sr + s * S1;
  const int64_t bm_seq = (a.nb + 1) * D * M, bc_seq = (a.nb + 1) * D * D;

  auto stage_piece = [&](int64_t ts, int len, bool with_grad) {
    const bool vec = a.vec && (ts % 4 == 0);
    stage_in<D, SUB, SPW>(sk, a.k, n0, a.n, T, ts, len, vec, lane);
    stage_in<M, SUB, SPW>(sv, a.v, n0, a.n, T, ts, len, vec, lane);
    stage_in<J, SUB, SPW>(srad, a.rad, n0, a.n, T, ts, len, vec, lane);
    stage_in<J, SUB, SPW>(sang, a.ang, n0, a.n, T, ts, len, vec, lane);
    stage_in<J, SUB, SPW>(sp, a.p, n0, a.n, T, ts, len, vec, lane);
    stage_in<1, SUB, SPW>(sr, a.r, n0, a.n, T, ts, len, vec, lane);
    if (with_grad) {
      stage_in<D, SUB, SPW>(sq, a.q, n0, a.n, T, ts, len, vec, lane);
      stage_in<M, SUB, SPW>(sg, a.gy, n0, a.n, T, ts, len, vec, lane);
    }
  };

  // Replay one piece (tokens [ts, ts + len) staged in the tiles) from belief
  // b with the history in registers, then reverse it; the gradients
  // overwrite the input tiles.
  auto replay_tok = [&](Belief<D, M, G>& b, const TokRot<D, M, G>& in, RotHist<D, M, G>& h)
      __attribute__((always_inline)) {
#pragma unroll
    for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
      for (int j = 0; j < D; ++j) h.Pp[jj][j] = b.P[jj][j];
#pragma unroll
    for (int i = 0; i < D; ++i)
#pragma unroll
      for (int cc = 0; cc < CPL; ++cc) h.Mp[i][cc] = b.Mv[i][cc];
    StepOut<D, M, G> o;
    float Pb[RPL][D];
    step_rot<D, M, G>(b, in, a.floor, g, lane, o, Pb);
#pragma unroll
    for (int j = 0; j < D; ++j) h.u[j] = o.u[j];
#pragma unroll
    for (int jj = 0; jj < RPL; ++jj) h.u_own[jj] = o.u_own[jj];
    h.s = o.s;
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) h.e[cc] = o.e[cc];
  };
  struct RevIn {
    TokRot<D, M, G> t;
    float q[D], gy[CPL];
  };
  auto read_rev = [&](RevIn& x, int tt) __attribute__((always_inline)) {
    read_rot<D, M, G>(x.t, st, tt, g, false);
#pragma unroll
    for (int j = 0; j < D; ++j) x.q[j] = gqs[tt * D + j];
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) x.gy[cc] = gys[tt * M + g * CPL + cc];
  };
  auto reverse_tok = [&](const RevIn& x, const RotHist<D, M, G>& h, int tt, int64_t ts)
      __attribute__((always_inline)) {
    RotOut<D, M, G> o;
    reverse_rot<D, M, G>(x.t, h, x.q, x.gy, gM, Gs, a.floor, g, lane, ts + tt == 0, gc0r, o);
    // Every lane has read its token inputs (the reads above and the
    // pair values inside) before any gradient overwrites them.
    __builtin_amdgcn_wave_barrier();
    if (writer) {
#pragma unroll
      for (int jj = 0; jj < RPL; ++jj) {
        const int rr = L::row(g, jj);
        gks[tt * D + rr] = o.gk_own[jj];
        gqs[tt * D + rr] = o.gq_own[jj];
      }
    }
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) gvs[tt * M + g * CPL + cc] = o.gv[cc];
    if (g == 0) {
#pragma unroll
      for (int m = 0; m < J; ++m) {
        grads[tt * J + m] = o.grad_rad[m];
        gangs[tt * J + m] = o.grad_ang[m];
        gps[tt * J + m] = o.gp[m];
      }
      grs[tt] = o.gr;
    }
  };
  auto run_piece = [&](Belief<D, M, G>& b, int64_t ts, int len) __attribute__((always_inline)) {
    RotHist<D, M, G> hist[SUB];
    if (len == SUB) {
      // A whole piece: each token's LDS reads are issued a token ahead (the
      // scheduling barriers keep them there), in both directions.
      TokRot<D, M, G> x[SUB];
      read_rot<D, M, G>(x[0], st, 0, g, true);
#pragma unroll
      for (int tt = 0; tt < SUB; ++tt) {
        if (tt + 1 < SUB) read_rot<D, M, G>(x[tt + 1], st, tt + 1, g, true);
        __builtin_amdgcn_sched_barrier(0);
        replay_tok(b, x[tt], hist[tt]);
        __builtin_amdgcn_sched_barrier(0);
      }
      RevIn r[SUB];
      read_rev(r[SUB - 1], SUB - 1);
#pragma unroll
      for (int tt = SUB - 1; tt >= 0; --tt) {
        if (tt > 0) read_rev(r[tt - 1], tt - 1);
        __builtin_amdgcn_sched_barrier(0);
        reverse_tok(r[tt], hist[tt], tt, ts);
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    }
#pragma unroll
    for (int tt = 0; tt < SUB; ++tt) {
      if (tt < len) {
        TokRot<D, M, G> in;
        read_rot<D, M, G>(in, st, tt, g, true);
        replay_tok(b, in, hist[tt]);
      }
    }
#pragma unroll
    for (int tt = SUB - 1; tt >= 0; --tt) {
      if (tt < len) {
        RevIn x;
        read_rev(x, tt);
        reverse_tok(x, hist[tt], tt, ts);
      }
    }
  };
  auto store_piece = [&](int64_t ts, int len) __attribute__((always_inline)) {
    const bool vec = a.vec && (ts % 4 == 0);
    stage_out<D, SUB, SPW>(sk, a.gk, n0, a.n, T, ts, len, vec, lane);
    stage_out<D, SUB, SPW>(sq, a.gq, n0, a.n, T, ts, len, vec, lane);
    stage_out<M, SUB, SPW>(sv, a.gv, n0, a.n, T, ts, len, vec, lane);
    stage_out<J, SUB, SPW>(srad, a.grad, n0, a.n, T, ts, len, vec, lane);
    stage_out<J, SUB, SPW>(sang, a.gang, n0, a.n, T, ts, len, vec, lane);
    stage_out<J, SUB, SPW>(sp, a.gp, n0, a.n, T, ts, len, vec, lane);
    stage_out<1, SUB, SPW>(sr, a.gr, n0, a.n, T, ts, len, vec, lane);
  };

  // Hot path (aligned streams, one replay piece per checkpoint chunk): the
  // next chunk (inputs and checkpoint records) lands in the staging area by
  // LDS-DMA while this one is computed; at a chunk's start the previous
  // chunk's gradients leave the tiles, then the staged rows are copied into
  // them.  Staging each chunk synchronously instead left the backward
  // waiting on memory for about a third of its time.
  const bool dma = a.vec && a.chunk == SUB && a.nb > 0 && T * 4 * M * SPW < (int64_t(1) << 31) &&
                   (a.nb + 1) * 4 * D * M * SPW < (int64_t(1) << 31);
  if (dma) {
    const uint32_t Tu = static_cast<uint32_t>(T);
    const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
    const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
    const r4::Rsrc xk = r4::make_rsrc(a.k + n0 * T * D, valid * Tu * D * 4u);
    const r4::Rsrc xq = r4::make_rsrc(a.q + n0 * T * D, valid * Tu * D * 4u);
    const r4::Rsrc xv = r4::make_rsrc(a.v + n0 * T * M, valid * Tu * M * 4u);
    const r4::Rsrc xg = r4::make_rsrc(a.gy + n0 * T * M, valid * Tu * M * 4u);
    const r4::Rsrc xrad = r4::make_rsrc(a.rad + n0 * T * J, valid * Tu * J * 4u);
    const r4::Rsrc xang = r4::make_rsrc(a.ang + n0 * T * J, valid * Tu * J * 4u);
    const r4::Rsrc xp = r4::make_rsrc(a.p + n0 * T * J, valid * Tu * J * 4u);
    const r4::Rsrc xr = r4::make_rsrc(a.r + n0 * T, valid * Tu * 4u);
    const r4::Rsrc xbm = r4::make_rsrc(a.bm + n0 * nbp * D * M, valid * nbp * D * M * 4u);
    const r4::Rsrc xbc = r4::make_rsrc(a.bc + n0 * nbp * D * D, valid * nbp * D * D * 4u);
    auto issue_dma = [&](int64_t c) {
      const uint32_t ts = static_cast<uint32_t>(c) * SUB, cu = static_cast<uint32_t>(c);
      dma_rows<SPW, SUB * D, D>(xk, stg + OK, Tu * D * 4u, ts * D * 4u, ts, Tu, lane);
      dma_rows<SPW, SUB * D, D>(xq, stg + OQ, Tu * D * 4u, ts * D * 4u, ts, Tu, lane);
      dma_rows<SPW, SUB * M, M>(xv, stg + OV, Tu * M * 4u, ts * M * 4u, ts, Tu, lane);
      dma_rows<SPW, SUB * M, M>(xg, stg + OG, Tu * M * 4u, ts * M * 4u, ts, Tu, lane);
      dma_rows<SPW, SUB * J, J>(xrad, stg + ORAD, Tu * J * 4u, ts * J * 4u, ts, Tu, lane);
      dma_rows<SPW, SUB * J, J>(xang, stg + OANG, Tu * J * 4u, ts * J * 4u, ts, Tu, lane);
      dma_rows<SPW, SUB * J, J>(xp, stg + OP, Tu * J * 4u, ts * J * 4u, ts, Tu, lane);
      dma_rows<SPW, SUB, 1>(xr, stg + OR, Tu * 4u, ts * 4u, ts, Tu, lane);
      dma_rows<SPW, D * M, 0>(xbm, stg + OBM, nbp * D * M * 4u, cu * D * M * 4u, 0, Tu, lane);
      dma_rows<SPW, D * D, 0>(xbc, stg + OBC, nbp * D * D * 4u, cu * D * D * 4u, 0, Tu, lane);
    };
    issue_dma(a.nb - 1);
    for (int64_t c = a.nb - 1; c >= 0; --c) {
      const int64_t ts = c * SUB;
      const int len = tile_len(T, ts, SUB);
      // Every outstanding memory operation was issued a whole chunk earlier.
      r4::vm_wait<0>();
      __syncthreads();
      if (c + 1 < a.nb) store_piece(ts + SUB, tile_len(T, ts + SUB, SUB));
      __syncthreads();
      copy_rows<SPW, D, SUB>(stg + OK, sk, lane);
      copy_rows<SPW, D, SUB>(stg + OQ, sq, lane);
      copy_rows<SPW, M, SUB>(stg + OV, sv, lane);
      copy_rows<SPW, M, SUB>(stg + OG, sg, lane);
      copy_rows<SPW, J, SUB>(stg + ORAD, srad, lane);
      copy_rows<SPW, J, SUB>(stg + OANG, sang, lane);
      copy_rows<SPW, J, SUB>(stg + OP, sp, lane);
      copy_rows<SPW, 1, SUB>(stg + OR, sr, lane);
      __syncthreads();
      fill_trig<SPW, J, SUB>(sang, ssi, lane);
      Belief<D, M, G> b;
#pragma unroll
      for (int i = 0; i < D; ++i)
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) b.Mv[i][cc] = active ? stg[OBM + s * D * M + i * M + g * CPL + cc] : 0.f;
#pragma unroll
      for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
        for (int j = 0; j < D; ++j)
          b.P[jj][j] = active ? stg[OBC + s * D * D + L::row(g, jj) * D + j] : (L::row(g, jj) == j ? 1.f : 0.f);
      __syncthreads();
      // The staging reads are complete before the next chunk's DMA lands.
      r4::lds_wait();
      if (c > 0) issue_dma(c - 1);
      run_piece(b, ts, len);
    }
    __syncthreads();
    store_piece(0, tile_len(T, 0, SUB));
  }


  for (int64_t c = dma ? -1 : a.nb - 1; c >= 0; --c) {
    const int64_t tc0 = c * a.chunk;
    const int64_t lc = (T - tc0) < a.chunk ? (T - tc0) : a.chunk;
    const int nsub = static_cast<int>((lc + SUB - 1) / SUB);
    for (int sc = nsub - 1; sc >= 0; --sc) {
      Belief<D, M, G> b;
      load_belief<D, M, G>(b, a.bm + na * bm_seq + c * D * M, a.bc + na * bc_seq + c * D * D, g, active);
      // Advance from the checkpoint to the piece.
      for (int j = 0; j < sc; ++j) {
        stage_piece(tc0 + static_cast<int64_t>(j) * SUB, SUB, false);
        __syncthreads();
        fill_trig<SPW, J, SUB>(sang, ssi, lane);
        __syncthreads();
#pragma unroll 1
        for (int tt = 0; tt < SUB; ++tt) {
          TokRot<D, M, G> in;
          read_rot<D, M, G>(in, st, tt, g, true);
          StepOut<D, M, G> o;
          float Pb[RPL][D];
          step_rot<D, M, G>(b, in, a.floor, g, lane, o, Pb);
        }
        __syncthreads();
      }
      const int64_t ts = tc0 + static_cast<int64_t>(sc) * SUB;
      const int len = static_cast<int>((lc - sc * SUB) < SUB ? (lc - sc * SUB) : SUB);
      stage_piece(ts, len, true);
      __syncthreads();
      fill_trig<SPW, J, SUB>(sang, ssi, lane);
      __syncthreads();
      run_piece(b, ts, len);
      __syncthreads();
      store_piece(ts, len);
      __syncthreads();
    }
  }

  if (active) {
    if (a.gm0) {
#pragma unroll
      for (int i = 0; i < D; ++i)
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) a.gm0[na * D * M + i * M + g * CPL + cc] = gM[i][cc];
    }
    if (a.gc0 && writer) {
#pragma unroll
      for (int jj = 0; jj < RPL; ++jj) {
        const int rr = L::row(g, jj);
#pragma unroll
        for (int j = 0; j < D; ++j) {
          const float raw = a.gcf ? a.gcf[na * D * D + rr * D + j] : 0.f;
          a.gc0[na * D * D + rr * D + j] = (T > 0) ? gc0r[jj][j] : raw;
        }
      }
    }
  }
}

template <int D>
struct RotTuning;
template <> struct RotTuning<2> { static constexpr int G = 4, TT = 16, SUB = 8; };
template <> struct RotTuning<4> { static constexpr int G = 4, TT = 16, SUB = 8; };
template <> struct RotTuning<8> { static constexpr int G = 8, TT = 16, SUB = 4; };

template <int D>
hipError_t fwd(const RotArgs& a, hipStream_t stream) {
  using Tn = RotTuning<D>;
  constexpr int SPW = kWave / Tn::G;
  const int64_t blocks = (a.n + SPW - 1) / SPW;
  hipLaunchKernelGGL((forward_kernel<D, 8, Tn::G, Tn::TT>), dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0,
                     stream, a);
  return hipGetLastError();
}
template <int D>
hipError_t bwd(const RotArgs& a, hipStream_t stream) {
  using Tn = RotTuning<D>;
  constexpr int SPW = kWave / Tn::G;
  const int64_t blocks = (a.n + SPW - 1) / SPW;
  hipLaunchKernelGGL((backward_kernel<D, 8, Tn::G, Tn::SUB>), dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace
}  // namespace rot

int rotation_checkpoint(int key_dim) {
  switch (key_dim) {
    case 2: return rot::RotTuning<2>::SUB;
    case 4: return rot::RotTuning<4>::SUB;
    case 8: return rot::RotTuning<8>::SUB;
    default: return 0;
  }
}

hipError_t launch_rotation_forward(int key_dim, const RotArgs& a, hipStream_t stream) {
  if (a.n == 0) return hipSuccess;
  auto al8 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; };
  if (key_dim == 4 && a.vec && a.t % 4 == 0 && a.n <= small_batch_limit(4) && al8(a.m0) && al8(a.mT) && al8(a.bm))
    return launch_rotation_forward_small(a, stream);
  switch (key_dim) {
    case 2: return rot::fwd<2>(a, stream);
    case 4: return rot::fwd<4>(a, stream);
    case 8: return rot::fwd<8>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rotation_backward(int key_dim, const RotArgs& a, hipStream_t stream) {
  if (a.n == 0) return hipSuccess;
  switch (key_dim) {
    case 2: return rot::bwd<2>(a, stream);
    case 4: return rot::bwd<4>(a, stream);
    case 8: return rot::bwd<8>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bssm
