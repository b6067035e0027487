// Static (A = I, Q = 0) associative scan in information form, gfx950.
//
// Equation reference: bayes_ssm/replay_ssm.py:251-270 and
// docs/associative_scan.md.  For every token t of batch row b:
//   L_t = inv(P0) + sum_{s<=t} k_s (k_s / r_s)^T
//   N_t = inv(P0) M0 + sum_{s<=t} (k_s / r_s) v_s^T
//   L_t <- (L_t + L_t^T) / 2,  M_t = L_t^{-1} N_t (Cholesky),  y_t = M_t^T q_t
// and for the last token also P_T = L_T^{-1}.
//
// Tokens are independent once their prefix is known, so the grid has one
// wave per (b, t).  The key dimension is a template parameter (runtime D is
// padded up to the next instantiated size: the padded block of every matrix
// is the identity and the padded key entries are zero, which leaves the
// leading block of every factor and solution unchanged).  Two lane roles:
//   row owners (lane i < D) hold row i of a D x D matrix in registers: the
//     prefix precision, then its Cholesky factor;
//   column owners (lane c < M) hold column c of the natural parameter and
//     solve for column c of the mean.
// The factorization broadcasts finished factor entries with readlane; the
// solves read the factor from LDS with uniform addresses (one 16-byte read
// serves four entries to every lane).  The prefix is summed sequentially
// over s (the association of a sequential cumsum); the token rows s are
// uniform across the wave and load as scalars.  Instantiated for D = 1, 2,
// 4, 8, 16; larger key dimensions (up to 32) take the LDS kernel below.

#include "bssm_recurrence.h"

namespace bssm {
namespace {

constexpr int kMaxD = 32;
constexpr int kMaxM = 64;

// Entry k of the row held by lane `row` (uniform row and k).
template <int D>
__device__ __forceinline__ float bcast(const float (&r)[D], int k, int row) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r[k]), row));
}

// Row-per-lane Cholesky: lane i < D holds row i of the SPD matrix A (lanes
// >= D hold zeros); on return it holds row i of the lower factor L (zeros
// above the diagonal) and inv_diag = 1 / L[i][i], and L is also in LDS
// (m, row-major) with its inverted diagonal in idg.  Each finished column is
// written to LDS, and column j reads the finished part of row j back with
// uniform addresses; only the pivot travels by readlane.
template <int D>
__device__ __forceinline__ void chol_rows(float (&a)[D], float& inv_diag, int lane, float* m, float* idg) {
#pragma unroll
  for (int j = 0; j < D; ++j) {
    float s = a[j];
#pragma unroll
    for (int k = 0; k < j; ++k) s = fmaf(-a[k], m[j * D + k], s);
    const float piv = sqrtf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), j)));
    const float rp = 1.0f / piv;
    a[j] = lane > j ? s * rp : (lane == j ? piv : 0.f);
    if (lane < D) m[lane * D + j] = a[j];
    if (lane == j) {
      inv_diag = rp;
      idg[j] = rp;
    }
  }
}

// Rows of a row-per-lane matrix into LDS (row-major, D x D), with the
// inverted diagonal of a factor in diag[] (only the first D lanes write).
template <int D>
__device__ __forceinline__ void rows_to_lds(const float (&a)[D], float* m, int lane) {
  if (lane < D) {
#pragma unroll
    for (int j = 0; j < D; j += 4) {
      v4f x;
      x[0] = a[j];
      x[1] = a[j + 1 < D ? j + 1 : j];
      x[2] = a[j + 2 < D ? j + 2 : j];
      x[3] = a[j + 3 < D ? j + 3 : j];
      if (j + 4 <= D) *reinterpret_cast<v4f*>(&m[lane * D + j]) = x;
      else
        for (int e = 0; e < D - j; ++e) m[lane * D + j + e] = x[e];
    }
  }
}

// Row i of an LDS matrix into registers (every lane reads the same words).
template <int D>
__device__ __forceinline__ void lds_row(const float* m, int i, float (&r)[D]) {
#pragma unroll
  for (int j = 0; j < D; j += 4) {
    if (j + 4 <= D) {
      const v4f x = *reinterpret_cast<const v4f*>(&m[i * D + j]);
      r[j] = x[0];
      r[j + 1] = x[1];
      r[j + 2] = x[2];
      r[j + 3] = x[3];
    } else {
      for (int e = 0; e < D - j; ++e) r[j + e] = m[i * D + j + e];
    }
  }
}

// Solve (L L^T) x = x in place for the calling lane's right-hand side; L
// (row-major) and 1 / diag(L) are in LDS and read with uniform addresses.
template <int D>
__device__ __forceinline__ void chol_solve(const float* L, const float* idg, float (&x)[D]) {
#pragma unroll
  for (int i = 0; i < D; ++i) {
    float li[D];
    lds_row<D>(L, i, li);
    float s = x[i];
#pragma unroll
    for (int k = 0; k < i; ++k) s = fmaf(-li[k], x[k], s);
    x[i] = s * idg[i];
  }
  // L^T x = z: column i of L is needed; rows k > i hold it at entry i.
#pragma unroll
  for (int i = D - 1; i >= 0; --i) {
    float s = x[i];
#pragma unroll
    for (int k = i + 1; k < D; ++k) s = fmaf(-L[k * D + i], x[k], s);
    x[i] = s * idg[i];
  }
}

// Padded (branch-free) element load: p[i] for i < n, else 0.
__device__ __forceinline__ float ld_or_zero(const float* p, int i, int n) {
  const float x = p[i < n ? i : 0];
  return i < n ? x : 0.f;
}

// The state of token t of batch row b, shared by the forward and the
// backward: on return the row owners hold row i of inv(P0) (lam0), LDS
// `mat` / `idg` hold the Cholesky factor of L_t and 1 / its diagonal, and the
// column owners hold column c of M_t = L_t^{-1} N_t in x.
template <int D, bool EXACT>
__device__ __forceinline__ void token_state(const float* __restrict__ keys, const float* __restrict__ values,
                                            const float* __restrict__ obs, const float* __restrict__ mean0,
                                            const float* __restrict__ cov0, int64_t T, int Dr, int M, int64_t b,
                                            int64_t t, int lane, float* mat, float* tr, float* idg,
                                            float (&lam0)[D], float (&x)[D]) {
  const bool row_lane = lane < Dr, col_lane = lane < M;
  const int rl = row_lane ? lane : 0, cl = col_lane ? lane : 0;

  // inv(P0): factor P0 (padded with the identity), then lane c < D solves for
  // column c of the identity; column c of inv(P0) is its row c (symmetric).
  float l[D], inv_diag = 1.f;
  const float* P0 = cov0 + (b * Dr + rl) * Dr;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const float v = ld_or_zero(P0, j, Dr);
    l[j] = row_lane ? v : (lane == j ? 1.f : 0.f);
  }
  chol_rows<D>(l, inv_diag, lane, mat, idg);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < D; ++j) lam0[j] = lane == j ? 1.f : 0.f;
  chol_solve<D>(mat, idg, lam0);
  __syncthreads();
  rows_to_lds<D>(lam0, mat, lane);  // mat = inv(P0)
  __syncthreads();

  // N_t column c starts at inv(P0) M0[:, c].
  float m0c[D];
  const float* M0 = mean0 + b * Dr * M + cl;
#pragma unroll
  for (int k = 0; k < D; ++k) {
    const float v = M0[(k < Dr ? k : 0) * M];
    m0c[k] = (col_lane && k < Dr) ? v : 0.f;
  }
#pragma unroll
  for (int i = 0; i < D; ++i) {
    float li[D];
    lds_row<D>(mat, i, li);
    float n0 = 0.f;
#pragma unroll
    for (int k = 0; k < D; ++k) n0 = fmaf(li[k], m0c[k], n0);
    x[i] = n0;
  }

  // Prefix sums over s <= t, in token order: row owners accumulate row i of
  // sum k (k / r)^T, column owners column c of sum (k / r) v^T.
  float acc[D];
#pragma unroll
  for (int j = 0; j < D; ++j) acc[j] = 0.f;
  const float* kb = keys + b * T * Dr;
  const float* vb = values + b * T * M + cl;
  const float* rb = obs + b * T;
#pragma unroll 4
  for (int64_t s = 0; s <= t; ++s) {
    float ks[D];
#pragma unroll
    for (int j = 0; j < D; ++j) ks[j] = ld_or_zero(kb + s * Dr, j, Dr);
    const float rinv = 1.0f / rb[s];
    const float kown = kb[s * Dr + rl], vown = vb[s * M];
    const float own = row_lane ? kown * rinv : 0.f;
    const float vc = col_lane ? vown : 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      acc[j] = fmaf(own, ks[j], acc[j]);
      x[j] = fmaf(ks[j] * rinv, vc, x[j]);
    }
  }

  // L_t = inv(P0) + prefix, symmetrized through LDS, on the row owners.
  // Padded rows (lanes Dr .. D - 1) keep the identity: lam0 there is the
  // identity row and acc is zero.
  float lam[D];
#pragma unroll
  for (int j = 0; j < D; ++j) lam[j] = lam0[j] + acc[j];
  if (lane < D) {
#pragma unroll
    for (int j = 0; j < D; ++j) tr[j * D + lane] = lam[j];
  }
  __syncthreads();
  if (lane < D) {
#pragma unroll
    for (int j = 0; j < D; ++j) lam[j] = (lam[j] + tr[lane * D + j]) * 0.5f;
  }
  float inv_lam = 1.f;
  __syncthreads();  // every lane is done with mat = inv(P0)
  chol_rows<D>(lam, inv_lam, lane, mat, idg);  // mat = factor of L_t
  __syncthreads();
  chol_solve<D>(mat, idg, x);
}

template <int D, bool EXACT>
__global__ __launch_bounds__(kWave) void associative_scan_kernel(const float* __restrict__ keys,
                                                                 const float* __restrict__ values,
                                                                 const float* __restrict__ queries,
                                                                 const float* __restrict__ obs,
                                                                 const float* __restrict__ mean0,
                                                                 const float* __restrict__ cov0,
                                                                 float* __restrict__ out, float* __restrict__ mT,
                                                                 float* __restrict__ cT, int64_t T, int Dr_, int M) {
  // EXACT: the runtime key dimension equals D (no padding masks at all).
  const int Dr = EXACT ? D : Dr_;
  __shared__ float mat[D * D];   // a factor or inv(P0), row-major
  __shared__ float tr[D * D];    // transpose staging for the symmetrization
  __shared__ float idg[D];       // 1 / diag of the factor in mat
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t t = blockIdx.x;
  const bool row_lane = lane < Dr, col_lane = lane < M;
  float lam0[D], x[D];
  token_state<D, EXACT>(keys, values, obs, mean0, cov0, T, Dr, M, b, t, lane, mat, tr, idg, lam0, x);

  const bool last = (t == T - 1);
  if (col_lane) {
    const float* qt = queries + (b * T + t) * Dr;
    float y = 0.f;
#pragma unroll
    for (int i = 0; i < D; ++i) y = fmaf(x[i], ld_or_zero(qt, i, Dr), y);
    out[(b * T + t) * M + lane] = y;
    if (last) {
#pragma unroll
      for (int i = 0; i < D; ++i)
        if (i < Dr) mT[(b * Dr + i) * M + lane] = x[i];
    }
  }
  if (last) {
    // P_T = L_T^{-1}: lane c solves for column c of the identity.
    float e[D];
#pragma unroll
    for (int i = 0; i < D; ++i) e[i] = lane == i ? 1.f : 0.f;
    chol_solve<D>(mat, idg, e);
    if (row_lane) {
#pragma unroll
      for (int i = 0; i < D; ++i)
        if (i < Dr) cT[(b * Dr + i) * Dr + lane] = e[i];
    }
  }
}

// ------------------------------------------------------------------ backward
// Reverse of the scan (the chain rule of replay_ssm.py:251-270).  With
// G_t = q_t gy_t^T (+ gM_T at the last token) the adjoint of M_t:
//   gq_t = M_t gy_t,   gN_t = L_t^{-1} G_t,
//   gL_t = sym(-gN_t M_t^T)  (+ sym(-P_T gP_T P_T) at the last token),
// where sym is the symmetrization the forward applies to L_t.  With the
// suffix sums SL_s = sum_{t>=s} gL_t and SN_s = sum_{t>=s} gN_t of the
// prefix terms k_s k_s^T / r_s and k_s v_s^T / r_s:
//   gk_s = (2 SL_s k_s + SN_s v_s) / r_s,   gv_s = SN_s^T k_s / r_s,
//   gr_s = -(k_s^T SL_s k_s + k_s^T SN_s v_s) / r_s^2,
// and for the prior (L_0 = inv(P0), N_0 = inv(P0) M0):
//   gM0 = inv(P0) SN_0,   gP0 = -inv(P0)^T (SL_0 + SN_0 M0^T) inv(P0)^T.
// Pass 1 (one wave per (b, t)) writes gq, gN_t and gL_t (workspace); pass 2
// turns the workspace into its suffix sums in place (one thread per entry of
// a batch row, tokens in reverse); pass 3 (one wave per (b, s)) forms the
// per-token gradients, and the s = 0 wave the prior's.
template <int D, bool EXACT>
__global__ __launch_bounds__(kWave) void scan_backward_token_kernel(
    const float* __restrict__ keys, const float* __restrict__ values, const float* __restrict__ queries,
    const float* __restrict__ obs, const float* __restrict__ mean0, const float* __restrict__ cov0,
    const float* __restrict__ gy, const float* __restrict__ gmT, const float* __restrict__ gcT,
    float* __restrict__ ws_gl, float* __restrict__ ws_gn, float* __restrict__ gq, int64_t T, int Dr_, int M) {
  const int Dr = EXACT ? D : Dr_;
  __shared__ float mat[D * D];
  __shared__ float tr[D * D];
  __shared__ float idg[D];
  __shared__ float mt[D * kMaxM];   // M_t, row-major
  __shared__ float gn[D * kMaxM];   // gN_t, row-major
  __shared__ float pt[D * D];       // P_T (last token), then P_T gP_T
  __shared__ float gys[kMaxM];
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t t = blockIdx.x;
  const bool row_lane = lane < Dr, col_lane = lane < M;
  float lam0[D], x[D];
  token_state<D, EXACT>(keys, values, obs, mean0, cov0, T, Dr, M, b, t, lane, mat, tr, idg, lam0, x);
  const bool last = (t == T - 1);
  const float* qt = queries + (b * T + t) * Dr;

  // Column owners: G[:, c] = q_t gy_t[c] (+ gM_T[:, c]), then gN[:, c] = L_t^{-1} G[:, c].
  float g[D];
  const float gyc = col_lane ? gy[(b * T + t) * M + lane] : 0.f;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    float v = ld_or_zero(qt, i, Dr) * gyc;
    if (last && gmT != nullptr && col_lane && i < Dr) v += gmT[(b * Dr + i) * M + lane];
    g[i] = col_lane ? v : 0.f;
  }
  chol_solve<D>(mat, idg, g);
  if (col_lane) {
    gys[lane] = gyc;
#pragma unroll
    for (int i = 0; i < D; ++i) {
      mt[i * kMaxM + lane] = x[i];
      gn[i * kMaxM + lane] = g[i];
      if (i < Dr) ws_gn[((b * T + t) * Dr + i) * M + lane] = g[i];
    }
  }
  // P_T for the last token's covariance adjoint.
  if (last && gcT != nullptr) {
    float e[D];
#pragma unroll
    for (int i = 0; i < D; ++i) e[i] = lane == i ? 1.f : 0.f;
    chol_solve<D>(mat, idg, e);  // lane c < D: column c of P_T (= row c)
    if (lane < D) {
#pragma unroll
      for (int i = 0; i < D; ++i) pt[lane * D + i] = e[i];
    }
  }
  __syncthreads();
  // Row owners: gq_t[i] = sum_c M_t[i, c] gy_t[c] and row i of -gN_t M_t^T.
  float gl[D];
  if (lane < D) {
    float acc = 0.f;
    for (int c = 0; c < M; ++c) acc = fmaf(mt[lane * kMaxM + c], gys[c], acc);
    if (row_lane) gq[(b * T + t) * Dr + lane] = acc;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      float a = 0.f;
      for (int c = 0; c < M; ++c) a = fmaf(gn[lane * kMaxM + c], mt[j * kMaxM + c], a);
      gl[j] = -a;
    }
  }
  if (last && gcT != nullptr && lane < D) {
    // -(P_T gP_T P_T)[i][:]: row i of A = P_T gP_T in registers, then A P_T
    // (gP_T and the padded block of P_T: zero and the identity).
    float a[D];
#pragma unroll
    for (int j = 0; j < D; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < D; ++k) {
        const float gkj = (k < Dr && j < Dr) ? gcT[(b * Dr + k) * Dr + j] : 0.f;
        acc = fmaf(pt[lane * D + k], gkj, acc);
      }
      a[j] = acc;
    }
#pragma unroll
    for (int j = 0; j < D; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < D; ++k) acc = fmaf(a[k], pt[k * D + j], acc);
      gl[j] -= acc;
    }
  }
  // Symmetrize through LDS and store row i of gL_t.
  __syncthreads();
  if (lane < D) {
#pragma unroll
    for (int j = 0; j < D; ++j) tr[j * D + lane] = gl[j];
  }
  __syncthreads();
  if (row_lane) {
#pragma unroll
    for (int j = 0; j < D; ++j)
      if (j < Dr) ws_gl[((b * T + t) * Dr + lane) * Dr + j] = (gl[j] + tr[lane * D + j]) * 0.5f;
  }
}

// Pass 2: ws rows [B, T, E] (E = D*D entries of gL_t, then D*M of gN_t, in
// their two arrays) to suffix sums over t >= s.  Loads run kSuffixBatch
// tokens ahead of the dependent sum.
constexpr int kSuffixBatch = 8;
__global__ __launch_bounds__(256) void scan_backward_suffix_kernel(float* __restrict__ ws_gl,
                                                                   float* __restrict__ ws_gn, int64_t T, int e_gl,
                                                                   int e_gn) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= e_gl + e_gn) return;
  const int64_t b = blockIdx.y;
  const bool gl = e < e_gl;
  const int w = gl ? e_gl : e_gn;
  float* p = (gl ? ws_gl + b * T * e_gl + e : ws_gn + b * T * e_gn + (e - e_gl));
  float acc = 0.f;
  int64_t t = T;
  while (t > 0) {
    const int n = t >= kSuffixBatch ? kSuffixBatch : static_cast<int>(t);
    float x[kSuffixBatch];
#pragma unroll
    for (int i = 0; i < kSuffixBatch; ++i) x[i] = i < n ? p[(t - 1 - i) * w] : 0.f;
#pragma unroll
    for (int i = 0; i < kSuffixBatch; ++i) {
      if (i < n) {
        acc += x[i];
        p[(t - 1 - i) * w] = acc;
      }
    }
    t -= n;
  }
}

template <int D, bool EXACT>
__global__ __launch_bounds__(kWave) void scan_backward_prefix_kernel(
    const float* __restrict__ keys, const float* __restrict__ values, const float* __restrict__ obs,
    const float* __restrict__ mean0, const float* __restrict__ cov0, const float* __restrict__ ws_gl,
    const float* __restrict__ ws_gn, float* __restrict__ gk, float* __restrict__ gv, float* __restrict__ gr,
    float* __restrict__ gm0, float* __restrict__ gc0, int64_t T, int Dr_, int M) {
  const int Dr = EXACT ? D : Dr_;
  __shared__ float mat[D * D];
  __shared__ float idg[D];
  __shared__ float sn[D * kMaxM];  // SN_s, row-major
  __shared__ float part[kWave];
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t s = blockIdx.x;
  const bool row_lane = lane < Dr, col_lane = lane < M;
  const int rl = row_lane ? lane : 0;
  // Suffix sums over t >= s (pass 2): row owners row i of SL, column owners column c of SN.
  float sl[D], snc[D];
  {
    const float* glt = ws_gl + ((b * T + s) * Dr + rl) * Dr;
    const float* gnt = ws_gn + (b * T + s) * Dr * M + (col_lane ? lane : 0);
#pragma unroll
    for (int j = 0; j < D; ++j) {
      sl[j] = (row_lane && j < Dr) ? glt[j < Dr ? j : 0] : 0.f;
      snc[j] = (col_lane && j < Dr) ? gnt[(j < Dr ? j : 0) * M] : 0.f;
    }
  }
  if (col_lane) {
#pragma unroll
    for (int i = 0; i < D; ++i) sn[i * kMaxM + lane] = snc[i];
  }
  __syncthreads();
  const float* ks = keys + (b * T + s) * Dr;
  const float* vs = values + (b * T + s) * M;
  const float rinv = 1.0f / obs[b * T + s];
  // gk_s[i] = (2 (SL k)_i + (SN v)_i) / r;  k^T SL k and k^T SN v for gr.
  float contrib = 0.f;
  if (row_lane) {
    float a = 0.f, n = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) a = fmaf(sl[j], ld_or_zero(ks, j, Dr), a);
    for (int c = 0; c < M; ++c) n = fmaf(sn[lane * kMaxM + c], vs[c], n);
    gk[(b * T + s) * Dr + lane] = (2.f * a + n) * rinv;
    contrib = ks[lane] * (a + n);
  }
  part[lane] = contrib;
  if (col_lane) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < D; ++i) a = fmaf(snc[i], ld_or_zero(ks, i, Dr), a);
    gv[(b * T + s) * M + lane] = a * rinv;
  }
  __syncthreads();
  if (lane == 0) {
    float z = 0.f;
    for (int i = 0; i < Dr; ++i) z += part[i];
    gr[b * T + s] = -z * rinv * rinv;
  }
  if (s != 0) return;
  // The prior: inv(P0) again (as in the forward), then
  // gM0 = inv(P0) SN_0 and gP0 = -inv(P0)^T (SL_0 + SN_0 M0^T) inv(P0)^T.
  float l[D], inv_diag = 1.f;
  const float* P0 = cov0 + (b * Dr + rl) * Dr;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const float v = ld_or_zero(P0, j, Dr);
    l[j] = row_lane ? v : (lane == j ? 1.f : 0.f);
  }
  __syncthreads();
  chol_rows<D>(l, inv_diag, lane, mat, idg);
  __syncthreads();
  float lam0[D];
#pragma unroll
  for (int j = 0; j < D; ++j) lam0[j] = lane == j ? 1.f : 0.f;
  chol_solve<D>(mat, idg, lam0);  // lane i < D: column i of inv(P0)
  __syncthreads();
  rows_to_lds<D>(lam0, mat, lane);  // mat = inv(P0)^T, row i = column i of inv(P0)
  __syncthreads();
  if (col_lane) {
    // gM0[i][c] = sum_k inv(P0)[i][k] SN[k][c]
#pragma unroll
    for (int i = 0; i < D; ++i) {
      float a = 0.f;
#pragma unroll
      for (int k = 0; k < D; ++k) a = fmaf(mat[k * D + i], snc[k], a);
      if (i < Dr) gm0[(b * Dr + i) * M + lane] = a;
    }
  }
  // gA = SL_0 + SN_0 M0^T (row owners, row i), then gP0 = -inv(P0)^T gA inv(P0)^T.
  float ga[D];
  if (lane < D) {
    const float* M0 = mean0 + b * Dr * M;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      float a = sl[j];
      if (row_lane && j < Dr)
        for (int c = 0; c < M; ++c) a = fmaf(sn[lane * kMaxM + c], M0[j * M + c], a);
      ga[j] = a;
    }
  }
  __syncthreads();
  float* tmp = sn;  // reuse: [D][D] rows of gA inv(P0)^T
  if (lane < D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      // (gA inv(P0)^T)[i][j] = sum_k gA[i][k] inv(P0)[j][k]
      float a = 0.f;
#pragma unroll
      for (int k = 0; k < D; ++k) a = fmaf(ga[k], mat[k * D + j], a);
      tmp[lane * D + j] = a;
    }
  }
  __syncthreads();
  if (row_lane) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      // gP0[i][j] = -sum_k inv(P0)[k][i] (gA inv(P0)^T)[k][j]
      float a = 0.f;
#pragma unroll
      for (int k = 0; k < D; ++k) a = fmaf(mat[lane * D + k], tmp[k * D + j], a);
      if (j < Dr) gc0[(b * Dr + lane) * Dr + j] = -a;
    }
  }
}

// Key dimensions 17..32: the general kernel with the matrices in LDS (a
// register-resident factor of that size would spill).  One wave per (b, t)
// as above; the factorization runs column by column in LDS.
// In-place Cholesky of the D x D matrix A (row-major in LDS); lower factor.
__device__ void lds_cholesky(float* A, int D, int lane) {
  for (int j = 0; j < D; ++j) {
    if (lane == 0) {
      float s = A[j * D + j];
      for (int k = 0; k < j; ++k) s = fmaf(-A[j * D + k], A[j * D + k], s);
      A[j * D + j] = sqrtf(s);
    }
    __syncthreads();
    const float piv = A[j * D + j];
    for (int i = j + 1 + lane; i < D; i += kWave) {
      float s = A[i * D + j];
      for (int k = 0; k < j; ++k) s = fmaf(-A[i * D + k], A[j * D + k], s);
      A[i * D + j] = s / piv;
    }
    __syncthreads();
  }
}

// Solve (L L^T) x = b for one right-hand side held by the calling lane.
__device__ void lds_chol_solve(const float* Lf, int D, float* x) {
  for (int i = 0; i < D; ++i) {
    float s = x[i];
    for (int k = 0; k < i; ++k) s = fmaf(-Lf[i * D + k], x[k], s);
    x[i] = s / Lf[i * D + i];
  }
  for (int i = D - 1; i >= 0; --i) {
    float s = x[i];
    for (int k = i + 1; k < D; ++k) s = fmaf(-Lf[k * D + i], x[k], s);
    x[i] = s / Lf[i * D + i];
  }
}

__global__ __launch_bounds__(kWave) void associative_scan_lds_kernel(const float* __restrict__ keys,
                                                                 const float* __restrict__ values,
                                                                 const float* __restrict__ queries,
                                                                 const float* __restrict__ obs,
                                                                 const float* __restrict__ mean0,
                                                                 const float* __restrict__ cov0,
                                                                 float* __restrict__ out, float* __restrict__ mT,
                                                                 float* __restrict__ cT, int64_t T, int D, int M) {
  __shared__ float C0[kMaxD * kMaxD];    // factor of P0
  __shared__ float Lam[kMaxD * kMaxD];   // precision, then its factor
  __shared__ float Nat[kMaxD * kMaxM];   // natural parameter
  __shared__ float Lam0[kMaxD * kMaxD];  // inv(P0)
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t t = blockIdx.x;
  const float* P0 = cov0 + b * D * D;
  const float* M0 = mean0 + b * D * M;

  // inv(P0) through its Cholesky factor (P0 is SPD).
  for (int e = lane; e < D * D; e += kWave) C0[e] = P0[e];
  __syncthreads();
  lds_cholesky(C0, D, lane);
  if (lane < D) {
    float x[kMaxD];
    for (int i = 0; i < D; ++i) x[i] = (i == lane) ? 1.f : 0.f;
    lds_chol_solve(C0, D, x);
    for (int i = 0; i < D; ++i) Lam0[i * D + lane] = x[i];
  }
  __syncthreads();

  // Prefix sums over s <= t, accumulated in token order.
  for (int e = lane; e < D * D; e += kWave) {
    const int i = e / D, j = e - i * D;
    float acc = 0.f;
    for (int64_t s = 0; s <= t; ++s) {
      const float* ks = keys + (b * T + s) * D;
      acc = fmaf(ks[i], ks[j] / obs[b * T + s], acc);
    }
    Lam[e] = Lam0[e] + acc;
  }
  for (int e = lane; e < D * M; e += kWave) {
    const int i = e / M, c = e - i * M;
    float acc = 0.f;
    for (int64_t s = 0; s <= t; ++s) {
      const float wk = keys[(b * T + s) * D + i] / obs[b * T + s];
      acc = fmaf(wk, values[(b * T + s) * M + c], acc);
    }
    float n0 = 0.f;
    for (int k = 0; k < D; ++k) n0 = fmaf(Lam0[i * D + k], M0[k * M + c], n0);
    Nat[e] = n0 + acc;
  }
  __syncthreads();
  // Symmetrise, then factor.
  for (int e = lane; e < D * D; e += kWave) {
    const int i = e / D, j = e - i * D;
    if (i < j) {
      const float v = (Lam[i * D + j] + Lam[j * D + i]) * 0.5f;
      Lam[i * D + j] = v;
      Lam[j * D + i] = v;
    }
  }
  __syncthreads();
  lds_cholesky(Lam, D, lane);

  const float* qt = queries + (b * T + t) * D;
  const bool last = (t == T - 1);
  for (int c = lane; c < M; c += kWave) {
    float x[kMaxD];
    for (int i = 0; i < D; ++i) x[i] = Nat[i * M + c];
    lds_chol_solve(Lam, D, x);
    float y = 0.f;
    for (int i = 0; i < D; ++i) y = fmaf(x[i], qt[i], y);
    out[(b * T + t) * M + c] = y;
    if (last)
      for (int i = 0; i < D; ++i) mT[b * D * M + i * M + c] = x[i];
  }
  if (last && lane < D) {
    float x[kMaxD];
    for (int i = 0; i < D; ++i) x[i] = (i == lane) ? 1.f : 0.f;
    lds_chol_solve(Lam, D, x);
    for (int i = 0; i < D; ++i) cT[b * D * D + i * D + lane] = x[i];
  }
}

// T == 0: the belief is the prior.
__global__ void copy_prior_kernel(const float* __restrict__ mean0, const float* __restrict__ cov0,
                                  float* __restrict__ mT, float* __restrict__ cT, int64_t nm, int64_t nc) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < nm) mT[i] = mean0[i];
  if (i < nc) cT[i] = cov0[i];
}

template <int D>
hipError_t launch_scan(const float* k, const float* v, const float* q, const float* r, const float* m0,
                       const float* c0, float* y, float* mT, float* cT, int64_t b, int64_t t, int d, int m,
                       hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(t), static_cast<unsigned>(b));
  if (d == D)
    hipLaunchKernelGGL((associative_scan_kernel<D, true>), grid, dim3(kWave), 0, stream, k, v, q, r, m0, c0, y, mT,
                       cT, t, d, m);
  else
    hipLaunchKernelGGL((associative_scan_kernel<D, false>), grid, dim3(kWave), 0, stream, k, v, q, r, m0, c0, y, mT,
                       cT, t, d, m);
  return hipGetLastError();
}

template <int D>
hipError_t launch_scan_backward(const float* k, const float* v, const float* q, const float* r, const float* m0,
                                const float* c0, const float* gy, const float* gmT, const float* gcT, float* ws,
                                float* gk, float* gv, float* gq, float* gr, float* gm0, float* gc0, int64_t b,
                                int64_t t, int d, int m, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(t), static_cast<unsigned>(b));
  float* ws_gl = ws;
  float* ws_gn = ws + b * t * d * d;
  if (d == D) {
    hipLaunchKernelGGL((scan_backward_token_kernel<D, true>), grid, dim3(kWave), 0, stream, k, v, q, r, m0, c0, gy,
                       gmT, gcT, ws_gl, ws_gn, gq, t, d, m);
  } else {
    hipLaunchKernelGGL((scan_backward_token_kernel<D, false>), grid, dim3(kWave), 0, stream, k, v, q, r, m0, c0, gy,
                       gmT, gcT, ws_gl, ws_gn, gq, t, d, m);
  }
  const int e_gl = d * d, e_gn = d * m;
  const dim3 sgrid(static_cast<unsigned>((e_gl + e_gn + 255) / 256), static_cast<unsigned>(b));
  hipLaunchKernelGGL(scan_backward_suffix_kernel, sgrid, dim3(256), 0, stream, ws_gl, ws_gn, t, e_gl, e_gn);
  if (d == D) {
    hipLaunchKernelGGL((scan_backward_prefix_kernel<D, true>), grid, dim3(kWave), 0, stream, k, v, r, m0, c0, ws_gl,
                       ws_gn, gk, gv, gr, gm0, gc0, t, d, m);
  } else {
    hipLaunchKernelGGL((scan_backward_prefix_kernel<D, false>), grid, dim3(kWave), 0, stream, k, v, r, m0, c0, ws_gl,
                       ws_gn, gk, gv, gr, gm0, gc0, t, d, m);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_associative_scan_backward(const float* k, const float* v, const float* q, const float* r,
                                            const float* m0, const float* c0, const float* gy, const float* gmT,
                                            const float* gcT, float* ws, float* gk, float* gv, float* gq, float* gr,
                                            float* gm0, float* gc0, int64_t b, int64_t t, int d, int m,
                                            hipStream_t stream) {
  if (d > kMaxBackwardD || m > kMaxM || d <= 0 || m <= 0 || t <= 0 || t > 0x7fffffff || b > 65535)
    return hipErrorInvalidValue;
  if (b == 0) return hipSuccess;
  if (d <= 1) return launch_scan_backward<1>(k, v, q, r, m0, c0, gy, gmT, gcT, ws, gk, gv, gq, gr, gm0, gc0, b, t, d, m, stream);
  if (d <= 2) return launch_scan_backward<2>(k, v, q, r, m0, c0, gy, gmT, gcT, ws, gk, gv, gq, gr, gm0, gc0, b, t, d, m, stream);
  if (d <= 4) return launch_scan_backward<4>(k, v, q, r, m0, c0, gy, gmT, gcT, ws, gk, gv, gq, gr, gm0, gc0, b, t, d, m, stream);
  if (d <= 8) return launch_scan_backward<8>(k, v, q, r, m0, c0, gy, gmT, gcT, ws, gk, gv, gq, gr, gm0, gc0, b, t, d, m, stream);
  return launch_scan_backward<16>(k, v, q, r, m0, c0, gy, gmT, gcT, ws, gk, gv, gq, gr, gm0, gc0, b, t, d, m, stream);
}

hipError_t launch_associative_scan(const float* k, const float* v, const float* q, const float* r,
                                   const float* m0, const float* c0, float* y, float* mT, float* cT,
                                   int64_t b, int64_t t, int d, int m, hipStream_t stream) {
  if (d > kMaxD || m > kMaxM || d <= 0 || m <= 0) return hipErrorInvalidValue;
  if (b == 0) return hipSuccess;
  if (t == 0) {
    const int64_t nm = b * d * m, nc = b * d * d;
    const int64_t total = nm > nc ? nm : nc;
    hipLaunchKernelGGL(copy_prior_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream,
                       m0, c0, mT, cT, nm, nc);
    return hipGetLastError();
  }
  if (t > 0x7fffffff || b > 65535) return hipErrorInvalidValue;
  if (d <= 1) return launch_scan<1>(k, v, q, r, m0, c0, y, mT, cT, b, t, d, m, stream);
  if (d <= 2) return launch_scan<2>(k, v, q, r, m0, c0, y, mT, cT, b, t, d, m, stream);
  if (d <= 4) return launch_scan<4>(k, v, q, r, m0, c0, y, mT, cT, b, t, d, m, stream);
  if (d <= 8) return launch_scan<8>(k, v, q, r, m0, c0, y, mT, cT, b, t, d, m, stream);
  if (d <= 16) return launch_scan<16>(k, v, q, r, m0, c0, y, mT, cT, b, t, d, m, stream);
  hipLaunchKernelGGL(associative_scan_lds_kernel, dim3(static_cast<unsigned>(t), static_cast<unsigned>(b)),
                     dim3(kWave), 0, stream, k, v, q, r, m0, c0, y, mT, cT, t, d, m);
  return hipGetLastError();
}

}  // namespace bssm
