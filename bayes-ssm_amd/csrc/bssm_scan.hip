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
// wave per (b, t): the prefix is summed directly (sequentially over s, the
// same association as a sequential cumsum), the D x D Cholesky factor is
// built in LDS column by column, and each lane solves one value column.
// The reference shapes (D <= 16, T <= 64) are launch-latency bound; this
// layout needs a single launch and no intermediate HBM tensors.

#include "bssm_recurrence.h"

namespace bssm {
namespace {

constexpr int kMaxD = 32;
constexpr int kMaxM = 64;

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
__device__ void chol_solve(const float* Lf, int D, float* x) {
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

__global__ __launch_bounds__(kWave) void associative_scan_kernel(const float* __restrict__ keys,
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
    chol_solve(C0, D, x);
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
    chol_solve(Lam, D, x);
    float y = 0.f;
    for (int i = 0; i < D; ++i) y = fmaf(x[i], qt[i], y);
    out[(b * T + t) * M + c] = y;
    if (last)
      for (int i = 0; i < D; ++i) mT[b * D * M + i * M + c] = x[i];
  }
  if (last && lane < D) {
    float x[kMaxD];
    for (int i = 0; i < D; ++i) x[i] = (i == lane) ? 1.f : 0.f;
    chol_solve(Lam, D, x);
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
  hipLaunchKernelGGL(associative_scan_kernel, dim3(static_cast<unsigned>(t), static_cast<unsigned>(b)), dim3(kWave),
                     0, stream, k, v, q, r, m0, c0, y, mT, cT, t, d, m);
  return hipGetLastError();
}

}  // namespace bssm
