// gfx950 kernels for the exact dense-covariance Bayesian recurrence with a
// diagonal transition (bayes_ssm/bayesian_layer.py:207-251 is the equation
// reference; bayes_ssm/fused_cuda.py:58-322 defines the extension contract).
//
// Per token, for one sequence (D key dims, M value columns):
//   P' = diag(d) P diag(d) + p I          u = P' k          s = r + k.u
//   beta = 1 / max(s, floor)              e = v - (d*M)^T k
//   M <- d*M + beta u e^T                 P <- P' - beta u u^T
//   y = M^T q
//
// Both kernels are persistent over the whole sequence: one launch per
// forward, one per backward.  A wave64 holds SPW = 64/G sequences (a group of
// G lanes per sequence, see bssm_common.h for the ownership rules).  Inputs
// are streamed through LDS tiles with coalesced 16-byte loads; the recurrent
// belief and its adjoint live in registers for the whole launch.
//
// The backward replays each checkpoint chunk (from bmean/bcov) on chip,
// keeping the replay history of up to SUB tokens in registers, then runs the
// reverse equations (bayes_ssm/persistent_bayes_chunked_d4m8.cu:291-343 for
// the reference conventions: asymmetric initial-covariance adjoint, strict
// s > floor gate on the observation gradient).  Chunks longer than SUB are
// split into SUB-token pieces, each replayed from the chunk start.
//
// The covariance stays bitwise symmetric: every update of entry (i, j) uses
// only commutative products (d_i*d_j, u_i*u_j), so the owner of row i and the
// owner of row j compute identical values.

#include <algorithm>

#include "bssm_step.h"

namespace bssm {

// ------------------------------------------------------------------ forward
template <int D, int M, int G, int TT, bool FIXED>
__global__ __launch_bounds__(kWave) void forward_kernel(FwdArgs a) {
  using L = Layout<D, M, G>;
  constexpr int SPW = L::SPW;
  constexpr int SD = Tile<D, TT>::STRIDE, SM = Tile<M, TT>::STRIDE, S1 = Tile<1, TT>::STRIDE;
  __shared__ float sk[SPW * SD];
  __shared__ float sq[SPW * SD];
  __shared__ float sv[SPW * SM];  // values in, readouts out (in place)
  __shared__ float sd[FIXED ? 1 : SPW * SD];
  __shared__ float sp[FIXED ? 1 : SPW * S1];
  __shared__ float sr[FIXED ? 1 : SPW * S1];

  const int lane = threadIdx.x;
  const int g = lane % G;
  const int s = lane / G;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t n = n0 + s;
  const bool active = n < a.n;
  const int64_t na = active ? n : 0;  // address index for idle lanes (never dereferenced)
  const int64_t T = a.t;

  float eye[L::RPL][D];
  init_eye<D, M, G>(eye, g);
  Belief<D, M, G> b;
  load_belief<D, M, G>(b, a.m0 + na * D * M, a.c0 + na * D * D, g, active);
  const int64_t bm_seq = (a.nb + 1) * D * M, bc_seq = (a.nb + 1) * D * D;
  if (active) store_belief<D, M, G>(b, a.bm + na * bm_seq, a.bc + na * bc_seq, g);

  SeqTile st;
  st.k = sk + s * SD;
  st.d = FIXED ? nullptr : sd + s * SD;
  st.v = sv + s * SM;
  st.p = FIXED ? nullptr : sp + s * S1;
  st.r = FIXED ? nullptr : sr + s * S1;
  const float* qs = sq + s * SD;
  float* ys = sv + s * SM;

  // All streams 16-byte aligned for every tile: register-staged loads with
  // the next tile in flight while this one is computed.  Otherwise scalar
  // staging per tile.
  const bool vec = a.vec_kqd && a.vec_v && a.vec_pr;
  TileRegs<D, TT, SPW> rk, rq, rd;
  TileRegs<M, TT, SPW> rv;
  TileRegs<1, TT, SPW> rp, rr;
  auto issue = [&](int64_t t0) {
    const int len = tile_len(T, t0, TT);
    rk.load(a.k, n0, a.n, T, t0, len, lane);
    rq.load(a.q, n0, a.n, T, t0, len, lane);
    rv.load(a.v, n0, a.n, T, t0, len, lane);
    if constexpr (!FIXED) {
      rd.load(a.d, n0, a.n, T, t0, len, lane);
      rp.load(a.p, n0, a.n, T, t0, len, lane);
      rr.load(a.r, n0, a.n, T, t0, len, lane);
    }
  };
  if (vec && T > 0) issue(0);

  int64_t next_ckpt = a.chunk;
  int64_t ckpt = 1;
  for (int64_t t0 = 0; t0 < T; t0 += TT) {
    const int len = tile_len(T, t0, TT);
    if (vec) {
      rk.commit(sk, lane);
      rq.commit(sq, lane);
      rv.commit(sv, lane);
      if constexpr (!FIXED) {
        rd.commit(sd, lane);
        rp.commit(sp, lane);
        rr.commit(sr, lane);
      }
    } else {
      stage_in_scalar<D, TT, SPW>(sk, a.k, n0, a.n, T, t0, len, lane);
      stage_in_scalar<D, TT, SPW>(sq, a.q, n0, a.n, T, t0, len, lane);
      stage_in_scalar<M, TT, SPW>(sv, a.v, n0, a.n, T, t0, len, lane);
      if constexpr (!FIXED) {
        stage_in_scalar<D, TT, SPW>(sd, a.d, n0, a.n, T, t0, len, lane);
        stage_in_scalar<1, TT, SPW>(sp, a.p, n0, a.n, T, t0, len, lane);
        stage_in_scalar<1, TT, SPW>(sr, a.r, n0, a.n, T, t0, len, lane);
      }
    }
    __syncthreads();
    if (vec && t0 + TT < T) issue(t0 + TT);
    // Software pipeline: the LDS reads of token tt+1 are issued before the
    // update of token tt, so their latency hides behind the arithmetic.
    TokenIn<D, M, G> cur;
    float qc[D];
    read_token<D, M, G, FIXED>(cur, st, 0, g, true);
#pragma unroll
    for (int j = 0; j < D; ++j) qc[j] = qs[j];
    for (int tt = 0; tt < len; ++tt) {
      const int nx = (tt + 1 < len) ? tt + 1 : tt;
      TokenIn<D, M, G> nxt;
      float qn[D];
      read_token<D, M, G, FIXED>(nxt, st, nx, g, true);
#pragma unroll
      for (int j = 0; j < D; ++j) qn[j] = qs[nx * D + j];
      if (t0 + tt == next_ckpt) {
        if (active)
          store_belief<D, M, G>(b, a.bm + na * bm_seq + ckpt * D * M, a.bc + na * bc_seq + ckpt * D * D, g);
        ++ckpt;
        next_ckpt += a.chunk;
      }
      StepOut<D, M, G> o;
      forward_step<D, M, G>(b, cur, eye, a.floor, lane, o);
#pragma unroll
      for (int c = 0; c < L::CPL; ++c) {
        float y = 0.f;
#pragma unroll
        for (int i = 0; i < D; ++i) y = fmaf(b.Mv[i][c], qc[i], y);
        ys[tt * M + g * L::CPL + c] = y;
      }
      cur = nxt;
#pragma unroll
      for (int j = 0; j < D; ++j) qc[j] = qn[j];
    }
    __syncthreads();
    stage_out<M, TT, SPW>(sv, a.y, n0, a.n, T, t0, len, vec, lane);
    __syncthreads();
  }
  if (active) {
    store_belief<D, M, G>(b, a.mT + na * D * M, a.cT + na * D * D, g);
    if (T > 0) store_belief<D, M, G>(b, a.bm + na * bm_seq + a.nb * D * M, a.bc + na * bc_seq + a.nb * D * D, g);
  }
}

// ----------------------------------------------------------------- backward
template <int D, int M, int G>
struct Hist {
  using L = Layout<D, M, G>;
  float Pp[L::RPL][D];   // covariance rows before the token
  float Mp[D][L::CPL];   // mean block before the token
  float u[D];
  float u_own[L::RPL];
  float s;
  float e[L::CPL];
};

template <int D, int M, int G, int SUB, bool FIXED, bool DYN>
__global__ __launch_bounds__(kWave) void backward_kernel(BwdArgs a) {
  using L = Layout<D, M, G>;
  constexpr int SPW = L::SPW, RPL = L::RPL, CPL = L::CPL;
  constexpr int SD = Tile<D, SUB>::STRIDE, SM = Tile<M, SUB>::STRIDE, S1 = Tile<1, SUB>::STRIDE;
  // keys/queries/decay/values/process/observation tiles are overwritten in
  // place by their gradients; sg holds the readout gradient.
  __shared__ float sk[SPW * SD];
  __shared__ float sq[SPW * SD];
  __shared__ float sd[SPW * SD];
  __shared__ float sv[SPW * SM];
  __shared__ float sg[SPW * SM];
  __shared__ float sp[SPW * S1];
  __shared__ float sr[SPW * S1];

  const int lane = threadIdx.x;
  const int g = lane % G;
  const int s = lane / G;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t n = n0 + s;
  const bool active = n < a.n;
  const int64_t na = active ? n : 0;  // address index for idle lanes (never dereferenced)
  const int64_t T = a.t;
  const bool writer = L::row_writer(g);

  float eye[RPL][D];
  init_eye<D, M, G>(eye, g);

  // Carried adjoints: gM = dL/dM (own columns), Gs = sym(dL/dP) (own rows).
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

  SeqTile st;
  st.k = sk + s * SD;
  st.d = sd + s * SD;
  st.v = sv + s * SM;
  st.p = sp + s * S1;
  st.r = sr + s * S1;
  float* gks = sk + s * SD;
  float* gqs = sq + s * SD;
  float* gds = sd + s * SD;
  float* gvs = sv + s * SM;
  const float* gys = sg + s * SM;
  float* gps = sp + s * S1;
  float* grs = sr + s * S1;

  const int64_t bm_seq = (a.nb + 1) * D * M, bc_seq = (a.nb + 1) * D * D;
  const bool vec_all = a.vec_kqd && a.vec_v && a.vec_pr;

  // Replay tokens [ts, ts + len) of the staged piece from belief b, keeping
  // the replay history in registers, then run the reverse over them; the
  // gradients overwrite the input tiles in LDS.
  auto run_piece = [&](Belief<D, M, G>& b, int64_t ts, int len) {
    Hist<D, M, G> h[SUB];
#pragma unroll
    for (int tt = 0; tt < SUB; ++tt) {
      if (tt < len) {
        TokenIn<D, M, G> in;
        read_token<D, M, G, FIXED>(in, st, tt, g, true);
#pragma unroll
        for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
          for (int j = 0; j < D; ++j) h[tt].Pp[jj][j] = b.P[jj][j];
#pragma unroll
        for (int i = 0; i < D; ++i)
#pragma unroll
          for (int cc = 0; cc < CPL; ++cc) h[tt].Mp[i][cc] = b.Mv[i][cc];
        StepOut<D, M, G> o;
        forward_step<D, M, G>(b, in, eye, a.floor, lane, o);
#pragma unroll
        for (int j = 0; j < D; ++j) h[tt].u[j] = o.u[j];
#pragma unroll
        for (int jj = 0; jj < RPL; ++jj) h[tt].u_own[jj] = o.u_own[jj];
        h[tt].s = o.s;
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) h[tt].e[cc] = o.e[cc];
      }
    }
#pragma unroll
    for (int tt = SUB - 1; tt >= 0; --tt) {
      if (tt < len) {
        TokenIn<D, M, G> in;
        read_token<D, M, G, FIXED>(in, st, tt, g, false);
        const Hist<D, M, G>& hh = h[tt];
        RevIn<D, M, G> x;
#pragma unroll
        for (int j = 0; j < D; ++j) x.q[j] = gqs[tt * D + j];
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) x.gy[cc] = gys[tt * M + g * CPL + cc];
        x.beta = fast_rcp(fmaxf(hh.s, a.floor));
        x.s = hh.s;
#pragma unroll
        for (int j = 0; j < D; ++j) x.u[j] = hh.u[j];
#pragma unroll
        for (int jj = 0; jj < RPL; ++jj) x.u_own[jj] = hh.u_own[jj];
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) x.e[cc] = hh.e[cc];
#pragma unroll
        for (int i = 0; i < D; ++i)
#pragma unroll
          for (int cc = 0; cc < CPL; ++cc) {
            x.Mprev[i][cc] = hh.Mp[i][cc];
            x.mp[i][cc] = in.d[i] * hh.Mp[i][cc];
          }
#pragma unroll
        for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
          for (int j = 0; j < D; ++j) {
            x.Pprev[jj][j] = hh.Pp[jj][j];
            x.Pb[jj][j] = fmaf(in.p, eye[jj][j], (in.d_own[jj] * in.d[j]) * hh.Pp[jj][j]);
          }
        RevOut<D, M, G> o;
        reverse_step<D, M, G, DYN>(in, x, gM, Gs, eye, a.floor, g, lane, ts + tt == 0, gc0r, o);
        if (writer) {
#pragma unroll
          for (int jj = 0; jj < RPL; ++jj) {
            const int rr = L::row(g, jj);
            gks[tt * D + rr] = o.gk_own[jj];
            gqs[tt * D + rr] = o.gq_own[jj];
            gds[tt * D + rr] = o.gd_own[jj];
          }
        }
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) gvs[tt * M + g * CPL + cc] = o.gv[cc];
        if (g == 0) {
          gps[tt] = o.gp;
          grs[tt] = o.gr;
        }
      }
    }
  };

  auto store_grads = [&](int64_t ts, int len, bool vec) {
    stage_out<D, SUB, SPW>(sk, a.gk, n0, a.n, T, ts, len, vec, lane);
    stage_out<D, SUB, SPW>(sq, a.gq, n0, a.n, T, ts, len, vec, lane);
    stage_out<M, SUB, SPW>(sv, a.gv, n0, a.n, T, ts, len, vec, lane);
    if (a.gd) stage_out<D, SUB, SPW>(sd, a.gd, n0, a.n, T, ts, len, vec, lane);
    if (a.gp) stage_out<1, SUB, SPW>(sp, a.gp, n0, a.n, T, ts, len, vec, lane);
    if (a.gr) stage_out<1, SUB, SPW>(sr, a.gr, n0, a.n, T, ts, len, vec, lane);
  };

  if (vec_all && a.chunk <= SUB && a.chunk % 4 == 0) {
    // Hot path: one replay piece per checkpoint chunk.  The inputs and the
    // checkpoint belief of chunk c-1 are loaded into registers while chunk c
    // is replayed and reversed.
    TileRegs<D, SUB, SPW> rk, rq, rd;
    TileRegs<M, SUB, SPW> rv, rg;
    TileRegs<1, SUB, SPW> rp, rr;
    Belief<D, M, G> nb_belief;
    auto issue = [&](int64_t c) {
      const int64_t ts = c * a.chunk;
      const int len = tile_len(T, ts, static_cast<int>(a.chunk));
      rk.load(a.k, n0, a.n, T, ts, len, lane);
      rq.load(a.q, n0, a.n, T, ts, len, lane);
      rv.load(a.v, n0, a.n, T, ts, len, lane);
      rg.load(a.gy, n0, a.n, T, ts, len, lane);
      if constexpr (!FIXED) {
        rd.load(a.d, n0, a.n, T, ts, len, lane);
        rp.load(a.p, n0, a.n, T, ts, len, lane);
        rr.load(a.r, n0, a.n, T, ts, len, lane);
      }
      load_belief<D, M, G>(nb_belief, a.bm + na * bm_seq + c * D * M, a.bc + na * bc_seq + c * D * D, g, active);
    };
    if (a.nb > 0) issue(a.nb - 1);
    for (int64_t c = a.nb - 1; c >= 0; --c) {
      const int64_t ts = c * a.chunk;
      const int len = tile_len(T, ts, static_cast<int>(a.chunk));
      rk.commit(sk, lane);
      rq.commit(sq, lane);
      rv.commit(sv, lane);
      rg.commit(sg, lane);
      if constexpr (!FIXED) {
        rd.commit(sd, lane);
        rp.commit(sp, lane);
        rr.commit(sr, lane);
      }
      Belief<D, M, G> b = nb_belief;
      __syncthreads();
      if (c > 0) issue(c - 1);
      run_piece(b, ts, len);
      __syncthreads();
      store_grads(ts, len, true);
      __syncthreads();
    }
  } else {
    // General path: chunks longer than SUB are replayed piece by piece from
    // their checkpoint; tiles are staged synchronously.
    for (int64_t c = a.nb - 1; c >= 0; --c) {
      const int64_t tc0 = c * a.chunk;
      const int64_t lc = (T - tc0) < a.chunk ? (T - tc0) : a.chunk;
      const int nsub = static_cast<int>((lc + SUB - 1) / SUB);
      for (int sc = nsub - 1; sc >= 0; --sc) {
        Belief<D, M, G> b;
        load_belief<D, M, G>(b, a.bm + na * bm_seq + c * D * M, a.bc + na * bc_seq + c * D * D, g, active);
        for (int j = 0; j < sc; ++j) {
          const int64_t ts = tc0 + static_cast<int64_t>(j) * SUB;
          const bool vec = vec_all && (ts % 4 == 0);
          stage_in<D, SUB, SPW>(sk, a.k, n0, a.n, T, ts, SUB, vec, lane);
          stage_in<M, SUB, SPW>(sv, a.v, n0, a.n, T, ts, SUB, vec, lane);
          if constexpr (!FIXED) {
            stage_in<D, SUB, SPW>(sd, a.d, n0, a.n, T, ts, SUB, vec, lane);
            stage_in<1, SUB, SPW>(sp, a.p, n0, a.n, T, ts, SUB, vec, lane);
            stage_in<1, SUB, SPW>(sr, a.r, n0, a.n, T, ts, SUB, vec, lane);
          }
          __syncthreads();
#pragma unroll 1
          for (int tt = 0; tt < SUB; ++tt) {
            TokenIn<D, M, G> in;
            read_token<D, M, G, FIXED>(in, st, tt, g, true);
            StepOut<D, M, G> o;
            forward_step<D, M, G>(b, in, eye, a.floor, lane, o);
          }
          __syncthreads();
        }
        const int64_t ts = tc0 + static_cast<int64_t>(sc) * SUB;
        const int len = static_cast<int>((lc - sc * SUB) < SUB ? (lc - sc * SUB) : SUB);
        const bool vec = vec_all && (ts % 4 == 0);
        stage_in<D, SUB, SPW>(sk, a.k, n0, a.n, T, ts, len, vec, lane);
        stage_in<D, SUB, SPW>(sq, a.q, n0, a.n, T, ts, len, vec, lane);
        stage_in<M, SUB, SPW>(sv, a.v, n0, a.n, T, ts, len, vec, lane);
        stage_in<M, SUB, SPW>(sg, a.gy, n0, a.n, T, ts, len, vec, lane);
        if constexpr (!FIXED) {
          stage_in<D, SUB, SPW>(sd, a.d, n0, a.n, T, ts, len, vec, lane);
          stage_in<1, SUB, SPW>(sp, a.p, n0, a.n, T, ts, len, vec, lane);
          stage_in<1, SUB, SPW>(sr, a.r, n0, a.n, T, ts, len, vec, lane);
        }
        __syncthreads();
        run_piece(b, ts, len);
        __syncthreads();
        store_grads(ts, len, vec);
        __syncthreads();
      }
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
          // With no tokens the adjoint passes through unchanged.
          const float raw = a.gcf ? a.gcf[na * D * D + rr * D + j] : 0.f;
          a.gc0[na * D * D + rr * D + j] = (T > 0) ? gc0r[jj][j] : raw;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ launch
namespace {

template <int D>
struct Tuning;
// G: lanes per sequence; TT: forward tile; SUB: replay piece (history in
// registers, so it scales inversely with the per-token history size).
template <> struct Tuning<1> { static constexpr int G = 8, TT = 32, SUB = 16; };
template <> struct Tuning<2> { static constexpr int G = 4, TT = 16, SUB = 8; };
template <> struct Tuning<4> { static constexpr int G = 4, TT = 16, SUB = 8; };
template <> struct Tuning<8> { static constexpr int G = 8, TT = 16, SUB = 8; };

template <int D, bool FIXED>
hipError_t launch_forward_d(const FwdArgs& a, hipStream_t stream) {
  using Tn = Tuning<D>;
  constexpr int SPW = kWave / Tn::G;
  const int64_t blocks = (a.n + SPW - 1) / SPW;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL((forward_kernel<D, 8, Tn::G, Tn::TT, FIXED>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kWave), 0, stream, a);
  return hipGetLastError();
}

template <int D, bool FIXED, bool DYN>
hipError_t launch_backward_d(const BwdArgs& a, hipStream_t stream) {
  using Tn = Tuning<D>;
  constexpr int SPW = kWave / Tn::G;
  const int64_t blocks = (a.n + SPW - 1) / SPW;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL((backward_kernel<D, 8, Tn::G, Tn::SUB, FIXED, DYN>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kWave), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

int preferred_checkpoint(int key_dim) {
  switch (key_dim) {
    case 1: return Tuning<1>::SUB;
    case 2: return Tuning<2>::SUB;
    case 4: return Tuning<4>::SUB;
    case 8: return Tuning<8>::SUB;
    case 64: return kD64Checkpoint;
    default: return 0;
  }
}

hipError_t launch_forward(int key_dim, bool fixed, const FwdArgs& a, hipStream_t stream) {
  // bf16 / float8 streams take the row kernels only within the two-wave
  // limit: above it their rotated-layout forward is the faster one.
  const int64_t row_limit = a.in_fmt == kInF32 ? small_batch_limit(0)
                                               : std::min(small_batch_limit(0), small_batch_limit(2));
  if (key_dim == 4 && a.rot4 && a.n <= row_limit) return launch_forward_small(fixed, a, stream);
  if (key_dim == 4 && a.rot4) return launch_forward_r4(fixed, a, stream);
  if (key_dim == 1 && d1_forward_ok(a)) return launch_forward_d1(fixed, a, stream);
  if (key_dim == 2 && d2_forward_ok(a)) return launch_forward_d2(fixed, a, stream);
  if (key_dim == 8 && d8_forward_ok(a)) return launch_forward_d8(fixed, a, stream);
  switch (key_dim) {
    case 1: return fixed ? launch_forward_d<1, true>(a, stream) : launch_forward_d<1, false>(a, stream);
    case 2: return fixed ? launch_forward_d<2, true>(a, stream) : launch_forward_d<2, false>(a, stream);
    case 4: return fixed ? launch_forward_d<4, true>(a, stream) : launch_forward_d<4, false>(a, stream);
    case 8: return fixed ? launch_forward_d<8, true>(a, stream) : launch_forward_d<8, false>(a, stream);
    case 64: return launch_forward_d64(fixed, a, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int D>
hipError_t launch_backward_dd(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  if (fixed) return launch_backward_d<D, true, false>(a, stream);
  return dyn ? launch_backward_d<D, false, true>(a, stream) : launch_backward_d<D, false, false>(a, stream);
}

hipError_t launch_backward(int key_dim, bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  // bf16 / float8 streams: only within the three-wave limit (as the forward).
  const int64_t row_limit = a.in_fmt == kInF32 ? small_batch_limit(1)
                                               : std::min(small_batch_limit(1), small_batch_limit(3));
  if (key_dim == 4 && a.rot4 && a.n <= row_limit && a.t % 16 == 0 && a.chunk == kRot4Chunk)
    return launch_backward_small(fixed, dyn, a, stream);
  if (key_dim == 4 && a.rot4) return launch_backward_r4(fixed, dyn, a, stream);
  if (key_dim == 1 && d1_backward_ok(a)) return launch_backward_d1(fixed, dyn, a, stream);
  if (key_dim == 2 && d2_backward_ok(a)) return launch_backward_d2(fixed, dyn, a, stream);
  if (key_dim == 8 && d8_backward_ok(a)) return launch_backward_d8(fixed, dyn, a, stream);
  switch (key_dim) {
    case 1: return launch_backward_dd<1>(fixed, dyn, a, stream);
    case 2: return launch_backward_dd<2>(fixed, dyn, a, stream);
    case 4: return launch_backward_dd<4>(fixed, dyn, a, stream);
    case 8: return launch_backward_dd<8>(fixed, dyn, a, stream);
    case 64: return launch_backward_d64(fixed, dyn, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bssm
