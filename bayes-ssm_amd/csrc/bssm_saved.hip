// Saved-history variant of the recurrence (the D1 ABI of the reference,
// bayes_ssm/persistent_bayes_chunked_d1m8.cu:387-414 and :466-650): the
// forward writes the exact per-token replay values to HBM and the reverse
// consumes them instead of replaying.  Same per-token math as the chunked
// kernels (bssm_step.h); inputs are read straight from global memory since
// this path trades bandwidth for skipping the replay and is not the tiled
// hot path.
//
// History layout (fp32, row-major): mp = d*M_prev [N,T,D,M], pp = P' [N,T,D,D],
// uh = u [N,T,D], bh = 1/max(s, floor) [N,T], eh = e [N,T,M].

#include "bssm_step.h"

namespace bssm {

template <int D, int M, int G>
__device__ __forceinline__ void read_token_global(TokenIn<D, M, G>& in, const FwdArgs& a, int64_t row, int g,
                                                  bool active) {
  using L = Layout<D, M, G>;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    in.k[j] = active ? a.k[row * D + j] : 0.f;
    in.d[j] = active ? a.d[row * D + j] : 1.f;
  }
#pragma unroll
  for (int jj = 0; jj < L::RPL; ++jj) {
    in.k_own[jj] = active ? a.k[row * D + L::row(g, jj)] : 0.f;
    in.d_own[jj] = active ? a.d[row * D + L::row(g, jj)] : 1.f;
  }
#pragma unroll
  for (int c = 0; c < L::CPL; ++c) in.v[c] = active ? a.v[row * M + g * L::CPL + c] : 0.f;
  in.p = active ? a.p[row] : 0.f;
  in.r = active ? a.r[row] : 1.f;
}

template <int D, int M, int G>
__global__ __launch_bounds__(kWave) void forward_saved_kernel(FwdArgs a, HistArgs h) {
  using L = Layout<D, M, G>;
  const int lane = threadIdx.x;
  const int g = lane % G;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * L::SPW + lane / G;
  const bool active = n < a.n;
  const int64_t na = active ? n : 0;  // address index for idle lanes (never dereferenced)
  const int64_t T = a.t;
  float eye[L::RPL][D];
  init_eye<D, M, G>(eye, g);
  Belief<D, M, G> b;
  load_belief<D, M, G>(b, a.m0 + na * D * M, a.c0 + na * D * D, g, active);
  const int64_t bm_seq = (a.nb + 1) * D * M, bc_seq = (a.nb + 1) * D * D;
  if (active) store_belief<D, M, G>(b, a.bm + na * bm_seq, a.bc + na * bc_seq, g);
  for (int64_t ti = 0; ti < T; ++ti) {
    const int64_t row = na * T + ti;
    TokenIn<D, M, G> in;
    read_token_global<D, M, G>(in, a, row, g, active);
    float Pprev[L::RPL][D];
#pragma unroll
    for (int jj = 0; jj < L::RPL; ++jj)
#pragma unroll
      for (int j = 0; j < D; ++j) Pprev[jj][j] = b.P[jj][j];
    if (active) {
#pragma unroll
      for (int i = 0; i < D; ++i)
#pragma unroll
        for (int c = 0; c < L::CPL; ++c) h.mp[(row * D + i) * M + g * L::CPL + c] = in.d[i] * b.Mv[i][c];
    }
    StepOut<D, M, G> o;
    forward_step<D, M, G>(b, in, eye, a.floor, lane, o);
    if (active) {
#pragma unroll
      for (int c = 0; c < L::CPL; ++c) {
        h.eh[row * M + g * L::CPL + c] = o.e[c];
        float y = 0.f;
#pragma unroll
        for (int i = 0; i < D; ++i) y = fmaf(b.Mv[i][c], a.q[row * D + i], y);
        a.y[row * M + g * L::CPL + c] = y;
      }
      if (L::row_writer(g)) {
#pragma unroll
        for (int jj = 0; jj < L::RPL; ++jj) {
          const int rr = L::row(g, jj);
          h.uh[row * D + rr] = o.u_own[jj];
#pragma unroll
          for (int j = 0; j < D; ++j)
            h.pp[(row * D + rr) * D + j] = fmaf(in.p, eye[jj][j], (in.d_own[jj] * in.d[j]) * Pprev[jj][j]);
        }
      }
      if (g == 0) h.bh[row] = fast_rcp(fmaxf(o.s, a.floor));
    }
  }
  if (active) {
    store_belief<D, M, G>(b, a.mT + na * D * M, a.cT + na * D * D, g);
    if (T > 0) store_belief<D, M, G>(b, a.bm + na * bm_seq + a.nb * D * M, a.bc + na * bc_seq + a.nb * D * D, g);
  }
}

template <int D, int M, int G, bool DYN>
__global__ __launch_bounds__(kWave) void backward_saved_kernel(BwdArgs a, HistArgs h) {
  using L = Layout<D, M, G>;
  constexpr int RPL = L::RPL, CPL = L::CPL;
  const int lane = threadIdx.x;
  const int g = lane % G;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * L::SPW + lane / G;
  const bool active = n < a.n;
  const int64_t na = active ? n : 0;  // address index for idle lanes (never dereferenced)
  const int64_t T = a.t;
  const bool writer = L::row_writer(g);
  float eye[RPL][D];
  init_eye<D, M, G>(eye, g);
  float gM[D][CPL], Gs[RPL][D], gc0r[RPL][D];
#pragma unroll
  for (int i = 0; i < D; ++i)
#pragma unroll
    for (int c = 0; c < CPL; ++c) gM[i][c] = (active && a.gmf) ? a.gmf[na * D * M + i * M + g * CPL + c] : 0.f;
#pragma unroll
  for (int jj = 0; jj < RPL; ++jj) {
    const int rr = L::row(g, jj);
#pragma unroll
    for (int j = 0; j < D; ++j) {
      Gs[jj][j] = (active && a.gcf) ? 0.5f * (a.gcf[na * D * D + rr * D + j] + a.gcf[na * D * D + j * D + rr]) : 0.f;
      gc0r[jj][j] = 0.f;
    }
  }
  const int64_t bm_seq = (a.nb + 1) * D * M, bc_seq = (a.nb + 1) * D * D;
  for (int64_t ti = T - 1; ti >= 0; --ti) {
    const int64_t row = na * T + ti;
    TokenIn<D, M, G> in;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      in.k[j] = active ? a.k[row * D + j] : 0.f;
      in.d[j] = active ? a.d[row * D + j] : 1.f;
    }
#pragma unroll
    for (int jj = 0; jj < RPL; ++jj) {
      in.k_own[jj] = active ? a.k[row * D + L::row(g, jj)] : 0.f;
      in.d_own[jj] = active ? a.d[row * D + L::row(g, jj)] : 1.f;
    }
    in.p = active ? a.p[row] : 0.f;
    in.r = active ? a.r[row] : 1.f;
    RevIn<D, M, G> x;
#pragma unroll
    for (int j = 0; j < D; ++j) x.q[j] = active ? a.q[row * D + j] : 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      x.gy[c] = active ? a.gy[row * M + g * CPL + c] : 0.f;
      x.e[c] = active ? h.eh[row * M + g * CPL + c] : 0.f;
    }
    x.beta = active ? h.bh[row] : 0.f;
    float s = in.r;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      x.u[j] = active ? h.uh[row * D + j] : 0.f;
      s = fmaf(in.k[j], x.u[j], s);
    }
    x.s = s;
#pragma unroll
    for (int jj = 0; jj < RPL; ++jj) x.u_own[jj] = active ? h.uh[row * D + L::row(g, jj)] : 0.f;
#pragma unroll
    for (int i = 0; i < D; ++i)
#pragma unroll
      for (int c = 0; c < CPL; ++c) x.mp[i][c] = active ? h.mp[(row * D + i) * M + g * CPL + c] : 0.f;
#pragma unroll
    for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
      for (int j = 0; j < D; ++j) x.Pb[jj][j] = active ? h.pp[(row * D + L::row(g, jj)) * D + j] : 0.f;
    // Belief before the token: the chunk checkpoint for token 0, otherwise
    // the posterior of the previous token rebuilt from its history.
    if (ti == 0) {
#pragma unroll
      for (int i = 0; i < D; ++i)
#pragma unroll
        for (int c = 0; c < CPL; ++c) x.Mprev[i][c] = active ? a.bm[na * bm_seq + i * M + g * CPL + c] : 0.f;
#pragma unroll
      for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
        for (int j = 0; j < D; ++j) x.Pprev[jj][j] = active ? a.bc[na * bc_seq + L::row(g, jj) * D + j] : 0.f;
    } else {
      const int64_t pr = row - 1;
      const float bp = active ? h.bh[pr] : 0.f;
      float up[D];
#pragma unroll
      for (int j = 0; j < D; ++j) up[j] = active ? h.uh[pr * D + j] : 0.f;
#pragma unroll
      for (int i = 0; i < D; ++i) {
        const float bu = bp * up[i];
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const float mpv = active ? h.mp[(pr * D + i) * M + g * CPL + c] : 0.f;
          const float ev = active ? h.eh[pr * M + g * CPL + c] : 0.f;
          x.Mprev[i][c] = fmaf(bu, ev, mpv);
        }
      }
#pragma unroll
      for (int jj = 0; jj < RPL; ++jj) {
        const int rr = L::row(g, jj);
        const float uo = active ? h.uh[pr * D + rr] : 0.f;
#pragma unroll
        for (int j = 0; j < D; ++j) {
          const float ppv = active ? h.pp[(pr * D + rr) * D + j] : 0.f;
          x.Pprev[jj][j] = fmaf(-bp, uo * up[j], ppv);
        }
      }
    }
    RevOut<D, M, G> o;
    reverse_step<D, M, G, DYN>(in, x, gM, Gs, eye, a.floor, g, lane, ti == 0, gc0r, o);
    if (active) {
      if (writer) {
#pragma unroll
        for (int jj = 0; jj < RPL; ++jj) {
          const int rr = L::row(g, jj);
          a.gk[row * D + rr] = o.gk_own[jj];
          a.gq[row * D + rr] = o.gq_own[jj];
          if (a.gd) a.gd[row * D + rr] = o.gd_own[jj];
        }
      }
#pragma unroll
      for (int c = 0; c < CPL; ++c) a.gv[row * M + g * CPL + c] = o.gv[c];
      if (g == 0) {
        if (a.gp) a.gp[row] = o.gp;
        if (a.gr) a.gr[row] = o.gr;
      }
    }
  }
  if (active) {
    if (a.gm0) {
#pragma unroll
      for (int i = 0; i < D; ++i)
#pragma unroll
        for (int c = 0; c < CPL; ++c) a.gm0[na * D * M + i * M + g * CPL + c] = gM[i][c];
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

namespace {
template <int D>
constexpr int saved_group() { return D == 1 ? 8 : (D == 8 ? 8 : 4); }

template <int D>
hipError_t fwd_saved_d(const FwdArgs& a, const HistArgs& h, hipStream_t stream) {
  constexpr int G = saved_group<D>();
  constexpr int SPW = kWave / G;
  const int64_t blocks = (a.n + SPW - 1) / SPW;
  hipLaunchKernelGGL((forward_saved_kernel<D, 8, G>), dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0, stream, a,
                     h);
  return hipGetLastError();
}

template <int D>
hipError_t bwd_saved_d(bool dyn, const BwdArgs& a, const HistArgs& h, hipStream_t stream) {
  constexpr int G = saved_group<D>();
  constexpr int SPW = kWave / G;
  const int64_t blocks = (a.n + SPW - 1) / SPW;
  if (dyn)
    hipLaunchKernelGGL((backward_saved_kernel<D, 8, G, true>), dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0,
                       stream, a, h);
  else
    hipLaunchKernelGGL((backward_saved_kernel<D, 8, G, false>), dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0,
                       stream, a, h);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_forward_saved(int key_dim, const FwdArgs& a, const HistArgs& h, hipStream_t stream) {
  switch (key_dim) {
    case 1: return fwd_saved_d<1>(a, h, stream);
    case 2: return fwd_saved_d<2>(a, h, stream);
    case 4: return fwd_saved_d<4>(a, h, stream);
    case 8: return fwd_saved_d<8>(a, h, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_backward_saved(int key_dim, bool dyn, const BwdArgs& a, const HistArgs& h, hipStream_t stream) {
  switch (key_dim) {
    case 1: return bwd_saved_d<1>(dyn, a, h, stream);
    case 2: return bwd_saved_d<2>(dyn, a, h, stream);
    case 4: return bwd_saved_d<4>(dyn, a, h, stream);
    case 8: return bwd_saved_d<8>(dyn, a, h, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bssm
