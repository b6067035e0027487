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
  float lam0[D];
#pragma unroll
  for (int j = 0; j < D; ++j) lam0[j] = lane == j ? 1.f : 0.f;
  chol_solve<D>(mat, idg, lam0);
  __syncthreads();
  rows_to_lds<D>(lam0, mat, lane);  // mat = inv(P0)
  __syncthreads();

  // N_t column c starts at inv(P0) M0[:, c].
  float x[D], m0c[D];
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

}  // namespace

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
