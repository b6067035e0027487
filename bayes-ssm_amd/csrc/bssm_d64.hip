// gfx950 kernels for D = M = 64 (bayes_ssm/persistent_bayes_chunked.cu is
// the reference extension for this shape: chunk_forward_kernel :175-261,
// recompute_chunk_kernel :263-301, backward_chunk_kernel :303-343).
//
// Two work decompositions share the per-token conventions below.
//
// Wave groups (the forward for every chunk, the backward at the preferred
// checkpoint interval kBlk = kD64Checkpoint = 8, bssm_recurrence.h): a
// workgroup of W waves per sequence, thread (w, l) holding 64 / W columns of
// covariance row l and the same rows of mean column l; row sums over j are W
// partial sums exchanged through LDS, sums over lanes go through a
// wave-private LDS transpose.  Inputs are staged per 8-token block through
// LDS.  The backward replays each chunk once, its history in registers.
//
// One wave per sequence (the backward at other chunks): lane l owns row l of
// the covariance P (P[j] = P_lj) and column l of the mean M (M[i] = M_il);
// every per-token matrix-vector product is a local 64-term dot product
// against a vector that all lanes read from LDS, and the reverse of token t
// replays from the chunk's checkpoint up to t (quadratic in the chunk
// length).  Row sums of mean-shaped products go through a padded 64 x 64 LDS
// transpose.
//
// Conventions: the covariance is carried as P~ + diag(pd): P~ collects the
// rank-one downdates and pd the process noise on the diagonal, so no lane
// has to address its own diagonal register (a run-time index) every token.
// Products that must commute (d_l d_j, u_l u_j, gu_l k_j + gu_j k_l) are
// formed without contraction, which keeps P and the covariance adjoint
// bitwise symmetric, as the reference's mirrored upper-triangle update does
// (persistent_bayes_chunked.cu:221-241).  Instead of the reference's
// per-token history in HBM (mp/pp/uh/bh/eh, 32 KB per token and sequence at
// D = 64), both backwards replay from the checkpoints on chip.

#include <type_traits>

#include "bssm_recurrence.h"
#include "bssm_rot4.h"
#include "bssm_step.h"

// No implicit contraction in this file: every fused multiply-add is an
// explicit fmaf, and every other product or sum is rounded on its own.  The
// all-reduce of s = r + k.u must not fuse its first sum with the product
// (each lane would round differently), and the commuted products that keep
// the covariance symmetric must round identically in both lanes.
#pragma clang fp contract(off)

namespace bssm {
namespace d64 {

constexpr int D = 64;

// Separately rounded products and sums (the file compiles without contraction).
__device__ __forceinline__ float mul_rn(float a, float b) { return a * b; }
__device__ __forceinline__ float add_rn(float a, float b) { return a + b; }

// Wave all-reduce with the bitwise-identical total in every lane: each step
// adds two commuted operands (quad xor 1, 2; half-row mirror; row mirror;
// xor 16; xor 32).
__device__ __forceinline__ float wave_sum(float x) {
  x = add_rn(x, dpp<kXor1>(x));
  x = add_rn(x, dpp<kXor2>(x));
  x = add_rn(x, dpp<kHalfMirror>(x));
  x = add_rn(x, dpp<0x140>(x));  // row_mirror: lane l <- 15 - l
  x = add_rn(x, __shfl_xor(x, 16, kWave));
  x = add_rn(x, __shfl_xor(x, 32, kWave));
  return x;
}

// Hand-off of LDS data between the lanes of the wave (a workgroup is one
// wave): the writes complete before any lane reads.
__device__ __forceinline__ void lds_handoff() { __syncthreads(); }

// Scheduling fence every 16 elements of a 64-long unrolled loop: bounds how
// many broadcast LDS reads the scheduler hoists ahead (register pressure).
__device__ __forceinline__ void quarter_fence(int j) {
  if (j != 0 && (j & 15) == 0) __builtin_amdgcn_sched_barrier(0);
}

// Dot product of the lane's 64 registers with a vector in LDS (all lanes read
// the same address: broadcast), four partial sums for instruction-level
// parallelism.
__device__ __forceinline__ float dot64(const float (&x)[D], const float* vec) {
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < D; j += 4) {
    quarter_fence(j);
    const v4f w = *reinterpret_cast<const v4f*>(&vec[j]);
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = fmaf(x[j + c], w[c], acc[c]);
  }
  return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// LDS rows of 64 floats padded to kRow: lane l's row starts at l * kRow, so
// the 16 lanes of one 16-byte access pass hit 16 distinct bank groups, and
// every chunk is an immediate offset from one base address per lane.
constexpr int kRow = D + 4;

// Column sum over lanes: lane l receives sum_r x^(r)[l] where x^(r) is lane
// r's register vector.  Lane r writes its vector as row r of a padded tile;
// lane l then reads element l of every row (64 consecutive words per row).
struct Transpose {
  // f(c) yields the lane's x[4c .. 4c+3].
  template <class F>
  __device__ __forceinline__ float sum(float* tile, int l, F&& f) const {
    float* row = tile + l * kRow;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      quarter_fence(4 * c);
      *reinterpret_cast<v4f*>(&row[4 * c]) = f(c);
    }
    lds_handoff();
    const float* col = tile + l;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < D; ++r) {
      quarter_fence(r);
      acc[r & 3] += col[r * kRow];
    }
    lds_handoff();  // every lane has read the tile before it is rewritten
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
};

// Per-lane token inputs.
struct Tok {
  float k, d, v, q, gy, p, r;
};

// The stream pointers are the sequence's rows (wave-uniform); t * D + l fits
// 32 bits (the C ABI bounds t * D by 2^25).
template <bool FIXED>
__device__ __forceinline__ Tok load_tok(const float* k, const float* v, const float* q, const float* d,
                                        const float* p, const float* r, const float* gy, int t, int l) {
  Tok x;
  const int e = t * D + l;
  x.k = k[e];
  x.v = v[e];
  x.q = q[e];
  x.gy = gy ? gy[e] : 0.f;
  if constexpr (FIXED) {
    x.d = kFixedDecay;
    x.p = kFixedProcess;
    x.r = kFixedObservation;
  } else {
    x.d = d[e];
    x.p = p[t];
    x.r = r[t];
  }
  return x;
}

// Broadcast vectors of the current token.
struct Bcast {
  float* k;
  float* d;
  float* q;
  float* wk;
  float* u;
  float* gu;
};

// Intermediates of one token: u_l = (P' k)_l, the unclamped innovation
// variance s, beta = 1 / max(s, floor) and the lane's innovation e_l.
struct Pred {
  float u, s, beta, e;
};

// Predict step of token x on the belief (P~ + diag(pd), M).  On the
// sequence's first token P holds the initial covariance row as given
// (possibly asymmetric), which u uses, as the reference does.
__device__ __forceinline__ Pred predict(const float (&P)[D], float pd, const float (&M)[D], const Tok& x, float floor,
                                        const Bcast& b, int l) {
  const float wk = x.d * x.k;
  b.k[l] = x.k;
  b.d[l] = x.d;
  b.q[l] = x.q;
  b.wk[l] = wk;
  lds_handoff();
  Pred o;
  float az[4] = {0.f, 0.f, 0.f, 0.f}, ae[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < D; j += 4) {
    quarter_fence(j);
    const v4f w = *reinterpret_cast<const v4f*>(&b.wk[j]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      az[c] = fmaf(P[j + c], w[c], az[c]);
      ae[c] = fmaf(M[j + c], w[c], ae[c]);
    }
  }
  const float z = fmaf(pd, wk, (az[0] + az[1]) + (az[2] + az[3]));
  o.u = fmaf(x.d, z, x.p * x.k);
  o.s = wave_sum(x.k * o.u) + x.r;
  o.beta = fast_rcp(fmaxf(o.s, floor));
  o.e = x.v - ((ae[0] + ae[1]) + (ae[2] + ae[3]));
  b.u[l] = o.u;
  lds_handoff();
  return o;
}

// Update step: M_il <- d_i M_il + u_i beta e_l,  P~_lj <- P~_lj d_l d_j -
// beta u_l u_j,  pd <- pd d_l^2 + p.  On the sequence's first token the
// covariance entries left of the diagonal are replaced by their mirrors
// (the initial covariance's upper triangle, read from `c0col`), as the
// reference writes the upper triangle and mirrors it.
__device__ __forceinline__ void update(float (&P)[D], float& pd, float (&M)[D], const Tok& x, const Pred& o,
                                       const Bcast& b, int l, const float* c0col) {
  const float be = o.beta * o.e;
  if (c0col) {
#pragma unroll
    for (int j = 0; j < D; ++j)
      if (j < l) P[j] = c0col[j * D];
    // The lane's diagonal entry is the as-given P0_ll either way.
  }
#pragma unroll
  for (int j = 0; j < D; j += 4) {
    quarter_fence(j);
    const v4f dv = *reinterpret_cast<const v4f*>(&b.d[j]);
    const v4f uv = *reinterpret_cast<const v4f*>(&b.u[j]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      M[j + c] = fmaf(uv[c], be, dv[c] * M[j + c]);
      P[j + c] = fmaf(-o.beta, mul_rn(o.u, uv[c]), P[j + c] * mul_rn(x.d, dv[c]));
    }
  }
  pd = fmaf(pd, mul_rn(x.d, x.d), x.p);
}

// P~ + diag(pd) as a plain row (diagonal folded in), for storing.
__device__ __forceinline__ float with_diag(const float (&P)[D], float pd, int j, int l) {
  return j == l ? P[j] + pd : P[j];
}

// ----------------------------------------------------------------- backward
// Reverse of one token (persistent_bayes_chunked.cu:303-343), lane l holding
// the belief before the token (P~, pd, M), its intermediates o, the carried
// adjoints S (row l of the symmetrized covariance adjoint, in LDS; Sd its
// diagonal entry) and gM (column l of the mean adjoint, in LDS like S).  `c0col` (first token only)
// points at column l of the initial covariance, whose upper triangle the
// predicted covariance of the first token mirrors.
struct RevOut {
  float gk, gq, gv, gd, gp, gr;
};

// Row l of the covariance adjoint and column l of the mean adjoint live in
// LDS (padded rows, see kRow): the replayed belief fills the register file.
__device__ __forceinline__ v4f& s_chunk(float* row, int c) { return *reinterpret_cast<v4f*>(&row[4 * c]); }

template <bool FIXED, bool DYN>
__device__ __forceinline__ RevOut reverse(const float (&P)[D], float pd, const float (&M)[D], const Tok& x,
                                          const Pred& o, float* srow, float& Sd, float* grow, float floor,
                                          const Bcast& b, float* tile, const Transpose& tr, int l,
                                          const float* c0col) {
  RevOut out;
  // dL/dM after the token includes q gy^T; ge = beta gM^T u.
  float gmu = 0.f;
  {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      quarter_fence(4 * c);
      const v4f qv = *reinterpret_cast<const v4f*>(&b.q[4 * c]);
      const v4f uv = *reinterpret_cast<const v4f*>(&b.u[4 * c]);
      v4f& gref = s_chunk(grow, c);
      v4f g4 = gref;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        g4[h] = fmaf(qv[h], x.gy, g4[h]);
        acc[h] = fmaf(g4[h], uv[h], acc[h]);
      }
      gref = g4;
    }
    gmu = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
  const float ge = o.beta * gmu;
  out.gv = ge;
  // dL/dq_i = sum_c M_new_ic gy_c with M_new = d M + beta u e^T.
  const float be = o.beta * o.e;
  out.gq = tr.sum(tile, l, [&](int c) __attribute__((always_inline)) {
    const v4f dv = *reinterpret_cast<const v4f*>(&b.d[4 * c]);
    const v4f uv = *reinterpret_cast<const v4f*>(&b.u[4 * c]);
    v4f r;
#pragma unroll
    for (int h = 0; h < 4; ++h) r[h] = fmaf(uv[h], be, dv[h] * M[4 * c + h]) * x.gy;
    return r;
  });
  // -sum_c (d M)_ic ge_c enters dL/dk_i.
  const float gk_mean = tr.sum(tile, l, [&](int c) __attribute__((always_inline)) {
    const v4f dv = *reinterpret_cast<const v4f*>(&b.d[4 * c]);
    v4f r;
#pragma unroll
    for (int h = 0; h < 4; ++h) r[h] = (dv[h] * M[4 * c + h]) * ge;
    return r;
  });
  // a_i = sum_c gM_ic e_c.
  const float a_l = tr.sum(tile, l, [&](int c) __attribute__((always_inline)) {
    return s_chunk(grow, c) * o.e;
  });
  // gM_prev = gM - k ge^T (its product with M_prev enters dL/dd); the
  // adjoint carried to the previous token is gM_prev * d.
  float gd_mean = 0.f;
  if constexpr (DYN) {
    gd_mean = tr.sum(tile, l, [&](int c) __attribute__((always_inline)) {
      const v4f kv = *reinterpret_cast<const v4f*>(&b.k[4 * c]);
      const v4f dv = *reinterpret_cast<const v4f*>(&b.d[4 * c]);
      v4f& gref = s_chunk(grow, c);
      v4f g4 = gref, r;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        g4[h] = fmaf(-kv[h], ge, g4[h]);
        r[h] = g4[h] * M[4 * c + h];
        g4[h] *= dv[h];
      }
      gref = g4;
      return r;
    });
  } else {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      quarter_fence(4 * c);
      const v4f kv = *reinterpret_cast<const v4f*>(&b.k[4 * c]);
      const v4f dv = *reinterpret_cast<const v4f*>(&b.d[4 * c]);
      v4f& gref = s_chunk(grow, c);
      v4f g4 = gref;
#pragma unroll
      for (int h = 0; h < 4; ++h) g4[h] = fmaf(-kv[h], ge, g4[h]) * dv[h];
      gref = g4;
    }
  }
  // w = S u, z = u.(a - w) summed over the wave.
  float w;
  {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      quarter_fence(4 * c);
      const v4f sv = s_chunk(srow, c);
      const v4f uv = *reinterpret_cast<const v4f*>(&b.u[4 * c]);
#pragma unroll
      for (int h = 0; h < 4; ++h) acc[h] = fmaf(sv[h], uv[h], acc[h]);
    }
    w = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
  const float z = wave_sum(fmaf(o.e, gmu, -(o.u * w)));
  const float gs = (o.s > floor) ? -z * o.beta * o.beta : 0.f;
  const float gu = fmaf(o.beta, fmaf(-2.f, w, a_l), gs * x.k);
  b.gu[l] = gu;
  lds_handoff();
  // dL/dk = -(dM) ge + gs u + P' gu, P' = (P~ + diag(pd)) d d^T + p I.
  float pgu;
  {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < D; j += 4) {
      quarter_fence(j);
      const v4f dv = *reinterpret_cast<const v4f*>(&b.d[j]);
      const v4f gv = *reinterpret_cast<const v4f*>(&b.gu[j]);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = fmaf(P[j + c] * mul_rn(x.d, dv[c]), gv[c], acc[c]);
    }
    pgu = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
  if (c0col != nullptr) {
    // First token: its predicted covariance mirrors P0's upper triangle, so
    // the entries left of the diagonal are P0_jl rather than the row's P0_lj.
    float corr = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const float dj = (j < l) ? (c0col[j * D] - P[j]) : 0.f;
      corr = fmaf(dj * mul_rn(x.d, b.d[j]), b.gu[j], corr);
    }
    pgu += corr;
  }
  out.gk = -gk_mean + fmaf(gs, o.u, fmaf(fmaf(pd, mul_rn(x.d, x.d), x.p), gu, pgu));
  // H = S + sym(gu k^T); dL/dd_l = 2 sum_j H_lj P_lj d_j + sum_c gM_prev_lc M_lc;
  // dL/dp = trace H; the adjoint before the token is H d d^T.
  float gd_cov = 0.f;
  const float hd = add_rn(Sd, 0.5f * add_rn(mul_rn(gu, x.k), mul_rn(gu, x.k)));
#pragma unroll
  for (int j = 0; j < D; j += 4) {
    quarter_fence(j);
    const v4f dv = *reinterpret_cast<const v4f*>(&b.d[j]);
    const v4f kv = *reinterpret_cast<const v4f*>(&b.k[j]);
    const v4f gv = *reinterpret_cast<const v4f*>(&b.gu[j]);
    v4f& sref = s_chunk(srow, j >> 2);
    const v4f sv = sref;
    v4f sn;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float h = add_rn(sv[c], 0.5f * add_rn(mul_rn(gu, kv[c]), mul_rn(gv[c], x.k)));
      if constexpr (DYN) gd_cov = fmaf(h * P[j + c], dv[c], gd_cov);
      sn[c] = h * mul_rn(x.d, dv[c]);
    }
    sref = sn;
  }
  Sd = hd * mul_rn(x.d, x.d);
  if constexpr (DYN) {
    gd_cov = fmaf(hd * pd, x.d, gd_cov);
    out.gd = fmaf(2.f, gd_cov, gd_mean);
    out.gp = wave_sum(hd);
    out.gr = gs;
  } else {
    out.gd = out.gp = out.gr = 0.f;
  }
  return out;
}

template <bool FIXED, bool DYN>
__global__ __launch_bounds__(kWave) void backward_kernel(BwdArgs a) {
  __shared__ float sk[D], sd[D], sq[D], swk[D], su[D], sgu[D];
  __shared__ float tile[D * kRow];
  __shared__ float sadj[D * kRow];  // covariance adjoint, row l at sadj + l * kRow
  __shared__ float gadj[D * kRow];  // mean adjoint, column l at gadj + l * kRow
  const Bcast b{sk, sd, sq, swk, su, sgu};
  const int l = threadIdx.x;
  const int64_t n = blockIdx.x;
  const int64_t T = a.t, nbp = a.nb + 1, chunk = a.chunk;
  const Transpose tr;
  const float* bm = a.bm + n * nbp * D * D;
  const float* bc = a.bc + n * nbp * D * D;
  const float* kp = a.k + n * T * D;
  const float* vp = a.v + n * T * D;
  const float* qp = a.q + n * T * D;
  const float* gyp = a.gy + n * T * D;
  const float* dp = FIXED ? nullptr : a.d + n * T * D;
  const float* pp = FIXED ? nullptr : a.p + n * T;
  const float* rp = FIXED ? nullptr : a.r + n * T;
  float* gkp = a.gk + n * T * D;
  float* gqp = a.gq + n * T * D;
  float* gvp = a.gv + n * T * D;
  float* gdp = a.gd ? a.gd + n * T * D : nullptr;
  float* gpp = a.gp ? a.gp + n * T : nullptr;
  float* grp = a.gr ? a.gr + n * T : nullptr;

  // Carried adjoints from the final-state gradients (null: zero).
  float* srow = sadj + l * kRow;
  float* grow = gadj + l * kRow;
  float Sd = 0.f;
  if (a.gmf) {
    const float* gmf = a.gmf + n * D * D;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      v4f gv;
#pragma unroll
      for (int h = 0; h < 4; ++h) gv[h] = gmf[(4 * c + h) * D + l];
      s_chunk(grow, c) = gv;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 16; ++c) s_chunk(grow, c) = v4f{0.f, 0.f, 0.f, 0.f};
  }
  if (a.gcf) {
    const float* gcf = a.gcf + n * D * D;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      v4f sv;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int j = 4 * c + h;
        sv[h] = 0.5f * (gcf[l * D + j] + gcf[j * D + l]);
      }
      s_chunk(srow, c) = sv;
    }
    Sd = 0.5f * (gcf[l * D + l] + gcf[l * D + l]);
  } else {
#pragma unroll
    for (int c = 0; c < 16; ++c) s_chunk(srow, c) = v4f{0.f, 0.f, 0.f, 0.f};
  }

  for (int64_t c = a.nb - 1; c >= 0; --c) {
    const int64_t t0 = c * chunk;
    const int64_t len = (T - t0) < chunk ? (T - t0) : chunk;
    for (int64_t tt = len - 1; tt >= 0; --tt) {
      // Belief before token t0 + tt: the checkpoint advanced tt tokens.
      float P[D], M[D];
      float pd = 0.f;
      const float* cm = bm + c * D * D;
      const float* cc = bc + c * D * D;
      // Row l (checkpoint 0 is the initial covariance as given, possibly
      // asymmetric; later checkpoints are symmetric).
#pragma unroll
      for (int j = 0; j < D; j += 4) {
        const v4f r4 = *reinterpret_cast<const v4f*>(&cc[l * D + j]);
#pragma unroll
        for (int h = 0; h < 4; ++h) P[j + h] = r4[h];
      }
#pragma unroll
      for (int i = 0; i < D; ++i) M[i] = cm[i * D + l];
      Tok nxt = load_tok<FIXED>(kp, vp, qp, dp, pp, rp, gyp, static_cast<int>(t0), l);
      int64_t j = 0;
      if (c == 0 && tt > 0) {  // the sequence's first token mirrors P0's upper triangle
        const Tok x = nxt;
        nxt = load_tok<FIXED>(kp, vp, qp, dp, pp, rp, gyp, 1, l);
        const Pred o = predict(P, pd, M, x, a.floor, b, l);
        update(P, pd, M, x, o, b, l, cc + l);
        j = 1;
      }
      for (; j < tt; ++j) {
        const Tok x = nxt;
        nxt = load_tok<FIXED>(kp, vp, qp, dp, pp, rp, gyp, static_cast<int>(t0 + j + 1), l);
        const Pred o = predict(P, pd, M, x, a.floor, b, l);
        update(P, pd, M, x, o, b, l, nullptr);
      }
      const int64_t t = t0 + tt;
      const Pred o = predict(P, pd, M, nxt, a.floor, b, l);
      const RevOut g = reverse<FIXED, DYN>(P, pd, M, nxt, o, srow, Sd, grow, a.floor, b, tile, tr, l,
                                           t == 0 ? a.c0 + n * D * D + l : nullptr);
      const int e = static_cast<int>(t) * D + l;
      gkp[e] = g.gk;
      gqp[e] = g.gq;
      gvp[e] = g.gv;
      if (gdp) gdp[e] = g.gd;
      if (l == 0) {
        if (gpp) gpp[t] = g.gp;
        if (grp) grp[t] = g.gr;
      }
    }
  }
  if (a.gm0) {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const v4f gv = s_chunk(grow, c);
#pragma unroll
      for (int h = 0; h < 4; ++h) a.gm0[n * D * D + (4 * c + h) * D + l] = gv[h];
    }
  }
  if (a.gc0) {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const v4f sv = s_chunk(srow, c);
#pragma unroll
      for (int h = 0; h < 4; ++h) a.gc0[n * D * D + (4 * c + h) * D + l] = sv[h];
    }
  }
}

// ------------------------------------------------ wave groups per sequence
// One workgroup of W waves per sequence (W = kForwardWaves in the forward,
// kBackwardWaves in the backward): thread (w, l)
// owns the KB = 64 / W columns J_w = [KB w, KB w + KB) of covariance row l
// (P~_lj, j in J_w) and the rows J_w of mean column l (M_il, i in J_w); the
// diagonal part pd_l and every per-lane scalar (u_l, s, e_l, ...) are
// carried by all W waves with identical bits.  Sums over j of a row
// (P~ wk, M^T wk, M^T q, ...) are W partial sums exchanged through LDS (one
// barrier) and added in the same order by every wave; sums over the lanes of
// a wave's KB rows go through a wave-private LDS transpose.  u_j and gu_j of
// J_w are read from their lanes (v_readlane).
//
// Inputs are staged per block of kBlk tokens in a double-buffered LDS stage,
// a block ahead, from which each lane reads its own entries and the wave's
// KB-wide slices (broadcast reads).  The forward loads the block's k, v, d, q
// rows into registers and writes them, with the rows of wk = d k, to the
// stage; the backward's k, v, q, gy, d rows go straight to the stage by
// LDS-DMA.  The backward checkpoints every kBlk tokens and keeps a whole
// chunk's replayed beliefs and intermediates in registers, so each token is
// replayed once.
//
// Waves per sequence: four in the forward (one wave per SIMD at 256
// sequences), eight in the backward (two per SIMD; its history of 8 tokens
// fits in 256 registers per lane only with 8-column blocks).
constexpr int kForwardWaves = 4;
constexpr int kBackwardWaves = 8;
constexpr int kBlk = 8;  // tokens per staged block and per backward chunk

typedef float v2f __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int wave_index() { return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)); }
__device__ __forceinline__ float lane_value(float x, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), src));
}

// x + (x of the lane 16 (32) apart), via the gfx950 row swaps: both
// registers of the swap are added, the same pair in every lane.  Written as
// inline assembly because this toolchain's optimizer folds the second result
// of __builtin_amdgcn_permlane{16,32}_swap into the first; the s_nop gives
// the swap the two wait states it needs after the VALU writes of its operands.
__device__ __forceinline__ float swap_add16(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}
__device__ __forceinline__ float swap_add32(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}
// Wave all-reduce with the same bits in every lane (no LDS traffic).
__device__ __forceinline__ float wave_total(float x) {
  x = add_rn(x, dpp<kXor1>(x));
  x = add_rn(x, dpp<kXor2>(x));
  x = add_rn(x, dpp<kHalfMirror>(x));
  x = add_rn(x, dpp<0x140>(x));  // row_mirror
  return swap_add32(swap_add16(x));
}

// Pairwise sum of the W waves' partials, the same order in every wave.
template <int W>
__device__ __forceinline__ float tree(const float (&x)[W]) {
  if constexpr (W == 4) return (x[0] + x[1]) + (x[2] + x[3]);
  else return ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
}

// Sum over the wave's 64 lanes of each of the lane's KB values x[ii]: the
// total of row ii lands in the G = 64 / KB lanes G ii .. G ii + G - 1.
// `tile` is wave-private, 64 rows of KB floats with the 16-byte pieces of row
// r permuted by tile_rot(r): the 16-byte row writes of any 8 (or 16)
// consecutive lanes then cover all 32 (64) banks, and the column reads of a
// row sum touch 64 consecutive words.  A wave's LDS operations complete in
// issue order, so no barrier separates the writes from the reads.
template <int KB>
__device__ __forceinline__ int tile_rot(int r) {
  return ((r >> 1) ^ (r >> 3)) & (KB / 4 - 1);
}
template <int KB>
__device__ __forceinline__ float lane_rowsum(float* tile, int l, const float (&x)[KB]) {
  constexpr int G = kWave / KB, NP = KB / 4;
  float* row = tile + l * KB;
  const int rot = tile_rot<KB>(l);
#pragma unroll
  for (int c = 0; c < NP; ++c)
    *reinterpret_cast<v4f*>(&row[4 * (c ^ rot)]) = v4f{x[4 * c], x[4 * c + 1], x[4 * c + 2], x[4 * c + 3]};
  __builtin_amdgcn_wave_barrier();
  const int ii = l / G, g = l % G;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < KB; ++m) {
    const int r = G * m + g;
    acc[m & 3] += tile[r * KB + 4 * ((ii >> 2) ^ tile_rot<KB>(r)) + (ii & 3)];
  }
  __builtin_amdgcn_wave_barrier();
  float t = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  t = add_rn(t, dpp<kXor1>(t));
  t = add_rn(t, dpp<kXor2>(t));
  if constexpr (G == 8) t = add_rn(t, dpp<kHalfMirror>(t));
  return t;
}

// LDS stage of one block (floats): rows of k, v, q, gy, d (kBlk x 64 each),
// then p and r of the block's tokens; the forward's stage also holds the
// rows of wk = d k (kSW).
constexpr int kSK = 0, kSV = kBlk * D, kSQ = 2 * kBlk * D, kSG = 3 * kBlk * D, kSD = 4 * kBlk * D;
constexpr int kSP = 5 * kBlk * D, kSR = kSP + kBlk, kStage = kSR + kBlk;
constexpr int kSW = kStage, kStageFwd = kSW + kBlk * D;
constexpr int kRowVecs = kBlk * D / 4;  // 16-byte pieces of one array's block

// The sequence's input streams.
struct Streams {
  const float *k, *v, *q, *gy, *d, *p, *r;
};

// The forward's block of staged inputs, held in registers between its load
// and its LDS write (loaded a block ahead).  Piece i of the block is array
// i / kRowVecs of k, v, d, q (k, v, q for fixed dynamics): with 256 threads
// the thread that holds a piece of k also holds the same piece of d, and
// writes their product to the wk rows.
template <int NT, bool FIXED>
struct Prefetch {
  static_assert(NT == 2 * kRowVecs, "k and d pieces in one thread");
  static constexpr int kArrays = FIXED ? 3 : 4;
  static constexpr int kVecs = kArrays * kRowVecs;
  static constexpr int kReps = (kVecs + NT - 1) / NT;
  v4f x[kReps];
  float s;

  __device__ __forceinline__ static int array_offset(int arr) {
    return arr == 0 ? kSK : arr == 1 ? kSV : (arr == 2 && !FIXED) ? kSD : kSQ;
  }
  __device__ __forceinline__ static const float* array_src(const Streams& sp, int arr) {
    return arr == 0 ? sp.k : arr == 1 ? sp.v : (arr == 2 && !FIXED) ? sp.d : sp.q;
  }
  // Loads of the block starting at token t0 (zeros past the end T).
  __device__ __forceinline__ void fetch(const Streams& sp, int t0, int T, int tid) {
#pragma unroll
    for (int rep = 0; rep < kReps; ++rep) {
      const int i = tid + rep * NT;
      if (kVecs % NT == 0 || i < kVecs) {
        const int arr = i / kRowVecs, o = (i % kRowVecs) * 4;
        const int t = t0 + o / D;
        x[rep] = t < T ? *reinterpret_cast<const v4f*>(array_src(sp, arr) + t0 * D + o) : v4f{0.f, 0.f, 0.f, 0.f};
      }
    }
    if (!FIXED && tid < 2 * kBlk) {
      const int t = t0 + tid % kBlk;
      s = t < T ? (tid < kBlk ? sp.p[t] : sp.r[t]) : 0.f;
    }
  }
  __device__ __forceinline__ void put(float* stage, int tid) const {
#pragma unroll
    for (int rep = 0; rep < kReps; ++rep) {
      const int i = tid + rep * NT;
      if (kVecs % NT == 0 || i < kVecs) {
        const int arr = i / kRowVecs, o = (i % kRowVecs) * 4;
        *reinterpret_cast<v4f*>(&stage[array_offset(arr) + o]) = x[rep];
      }
    }
    if (tid < kRowVecs) {  // x[0] is a piece of k; x[1] the same piece of d
      const v4f dv = FIXED ? v4f{kFixedDecay, kFixedDecay, kFixedDecay, kFixedDecay} : x[1];
      *reinterpret_cast<v4f*>(&stage[kSW + 4 * tid]) = v4f{dv[0] * x[0][0], dv[1] * x[0][1], dv[2] * x[0][2],
                                                           dv[3] * x[0][3]};
    }
    if (!FIXED && tid < 2 * kBlk) stage[kSP + tid] = s;
  }
};

// The backward's block loads go straight from global memory into the stage
// (buffer_load ... lds): the rows of k, v, q, gy and d of the block starting
// at token t0, 16 bytes per lane, past the end T read as zeros by the
// descriptor's range check.  Nothing is held in registers while they are in
// flight; the issuing wave awaits them with a vmcnt wait before the barrier
// that publishes the stage.  p and r (8 floats each) go through the
// registers of threads 0 .. 2 kBlk - 1 (dma_pr / put_pr).
template <int NT, bool FIXED>
__device__ __forceinline__ void stage_dma(const Streams& sp, float* stage, int t0, int T, int tid) {
  constexpr int kArrays = 4 + (FIXED ? 0 : 1);
  constexpr int kVecs = kArrays * kRowVecs;
  const uint32_t bytes = static_cast<uint32_t>(T) * D * 4;
#pragma unroll
  for (int rep = 0; rep < (kVecs + NT - 1) / NT; ++rep) {
    const int i0 = __builtin_amdgcn_readfirstlane((tid & ~(kWave - 1)) + rep * NT);  // the wave's first piece
    if (kVecs % NT == 0 || i0 < kVecs) {
      const int arr = i0 / kRowVecs, o = (i0 % kRowVecs) * 4;
      const float* src = arr == 0 ? sp.k : arr == 1 ? sp.v : arr == 2 ? sp.q : arr == 3 ? sp.gy : sp.d;
      const int off = arr == 0 ? kSK : arr == 1 ? kSV : arr == 2 ? kSQ : arr == 3 ? kSG : kSD;
      r4::dma16<true>(r4::make_rsrc(src, bytes), stage + off + o,
                      static_cast<uint32_t>(t0 * D + o + 4 * (tid & (kWave - 1))) * 4u);
    }
  }
}
__device__ __forceinline__ float dma_pr(const Streams& sp, int t0, int T, int tid) {
  const int t = t0 + tid % kBlk;
  return t < T ? (tid < kBlk ? sp.p[t] : sp.r[t]) : 0.f;
}

// One token's inputs for thread (w, l): the lane's entries and the wave's
// KB-wide slices.
template <int KB>
struct TokG {
  float k, d, v, q, gy, p, r;
  float kJ[KB], dJ[KB], qJ[KB], wJ[KB];  // wJ = dJ kJ
};

// WK: the stage holds the wk rows (forward); otherwise wJ is formed here
// (the same single rounding).
template <int KB, bool FIXED, bool GY, bool WK = false>
__device__ __forceinline__ void read_tok(TokG<KB>& x, const float* st, int tt, int l, int j0) {
  const int e = tt * D + l, b = tt * D + j0;
  x.k = st[kSK + e];
  x.v = st[kSV + e];
  x.q = st[kSQ + e];
  x.gy = GY ? st[kSG + e] : 0.f;
#pragma unroll
  for (int c = 0; c < KB / 4; ++c) {
    const v4f kv = *reinterpret_cast<const v4f*>(&st[kSK + b + 4 * c]);
    const v4f qv = *reinterpret_cast<const v4f*>(&st[kSQ + b + 4 * c]);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      x.kJ[4 * c + h] = kv[h];
      x.qJ[4 * c + h] = qv[h];
    }
  }
  if constexpr (FIXED) {
    x.d = kFixedDecay;
    x.p = kFixedProcess;
    x.r = kFixedObservation;
#pragma unroll
    for (int jj = 0; jj < KB; ++jj) x.dJ[jj] = kFixedDecay;
  } else {
    x.d = st[kSD + e];
    x.p = st[kSP + tt];
    x.r = st[kSR + tt];
#pragma unroll
    for (int c = 0; c < KB / 4; ++c) {
      const v4f dv = *reinterpret_cast<const v4f*>(&st[kSD + b + 4 * c]);
#pragma unroll
      for (int h = 0; h < 4; ++h) x.dJ[4 * c + h] = dv[h];
    }
  }
  if constexpr (WK) {
#pragma unroll
    for (int c = 0; c < KB / 4; ++c) {
      const v4f wv = *reinterpret_cast<const v4f*>(&st[kSW + b + 4 * c]);
#pragma unroll
      for (int h = 0; h < 4; ++h) x.wJ[4 * c + h] = wv[h];
    }
  } else {
#pragma unroll
    for (int jj = 0; jj < KB; ++jj) x.wJ[jj] = x.dJ[jj] * x.kJ[jj];
  }
}

// Belief block of thread (w, l).
template <int KB>
struct BelG {
  float P[KB];  // P~_lj, j in J_w
  float M[KB];  // M_il, i in J_w
  float pd;
};

// A token's intermediates: u_l, beta = 1 / max(s, floor) and e_l; `clamped`
// records s <= floor (no gradient through s).
struct PredG {
  float u, beta, e;
  bool clamped;
};

// Partial sums of the predict step over the wave's block: (P~ wk)_l, (M^T wk)_l.
template <int KB>
__device__ __forceinline__ v2f predict_part(const BelG<KB>& b, const TokG<KB>& x) {
  float az[4] = {0.f, 0.f, 0.f, 0.f}, ae[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int jj = 0; jj < KB; ++jj) {
    az[jj & 3] = fmaf(b.P[jj], x.wJ[jj], az[jj & 3]);
    ae[jj & 3] = fmaf(b.M[jj], x.wJ[jj], ae[jj & 3]);
  }
  return v2f{(az[0] + az[1]) + (az[2] + az[3]), (ae[0] + ae[1]) + (ae[2] + ae[3])};
}

// u_l, beta, e_l from the W waves' partial sums zs (of P~ wk) and es (of M^T wk).
template <int W, int KB>
__device__ __forceinline__ PredG predict_done(const BelG<KB>& b, const TokG<KB>& x, const float (&zs)[W],
                                              const float (&es)[W], float floor) {
  const float z = fmaf(b.pd, x.d * x.k, tree<W>(zs));
  PredG o;
  o.u = fmaf(x.d, z, x.p * x.k);
  const float s = wave_total(x.k * o.u) + x.r;
  o.clamped = !(s > floor);
  o.beta = fast_rcp(fmaxf(s, floor));
  o.e = x.v - tree<W>(es);
  return o;
}

// Update of the block: M_il <- d_i M_il + u_i beta e_l, P~_lj <- P~_lj d_l d_j
// - beta u_l u_j, pd <- pd d_l^2 + p.  The rank-one terms are formed from
// g = sqrt(beta) u as one fused multiply-add, fma(-g_l, g_j, P~_lj d_l d_j),
// whose exact product commutes, so the covariance stays bitwise symmetric.
// On the sequence's first token the entries left of the diagonal are first
// replaced by their mirrors P0_jl (c0col: column l of the initial covariance).
template <int KB>
__device__ __forceinline__ void update_g(BelG<KB>& b, const TokG<KB>& x, const PredG& o, int l, int j0,
                                         const float* c0col) {
  if (c0col) {
#pragma unroll
    for (int jj = 0; jj < KB; ++jj)
      if (j0 + jj < l) b.P[jj] = c0col[(j0 + jj) * D];
  }
  const float rb = __builtin_amdgcn_sqrtf(o.beta);
  const float gl = rb * o.u, ge = rb * o.e;
#pragma unroll
  for (int jj = 0; jj < KB; ++jj) {
    const float gj = lane_value(gl, j0 + jj);
    b.M[jj] = fmaf(gj, ge, x.dJ[jj] * b.M[jj]);
    b.P[jj] = fmaf(-gl, gj, b.P[jj] * mul_rn(x.d, x.dJ[jj]));
  }
  b.pd = fmaf(b.pd, mul_rn(x.d, x.d), x.p);
}

template <int W, bool FIXED>
__global__ __launch_bounds__(W * kWave) void forward_group_kernel(FwdArgs a) {
  constexpr int KB = D / W, NT = W * kWave;
  // Exchange of {P~ wk, M^T wk, M^T q of the previous token} partials,
  // double-buffered: one barrier per token.
  __shared__ v4f xz[2][W * kWave];
  __shared__ __attribute__((aligned(16))) float stage[2][kStageFwd];
  const int tid = static_cast<int>(threadIdx.x), w = wave_index(), l = tid & (kWave - 1), j0 = KB * w;
  const int64_t n = blockIdx.x;
  const int T = static_cast<int>(a.t);
  const int64_t nbp = a.nb + 1;
  const float* c0 = a.c0 + n * D * D;
  const float* m0 = a.m0 + n * D * D;
  float* bm = a.bm + n * nbp * D * D;
  float* bc = a.bc + n * nbp * D * D;
  const Streams sp{a.k + n * T * D, a.v + n * T * D, a.q + n * T * D, nullptr,
                   FIXED ? nullptr : a.d + n * T * D, FIXED ? nullptr : a.p + n * T, FIXED ? nullptr : a.r + n * T};
  float* yp = a.y + n * T * D;

  BelG<KB> b;
  b.pd = 0.f;
#pragma unroll
  for (int c = 0; c < KB / 4; ++c) {
    const v4f r4 = *reinterpret_cast<const v4f*>(&c0[l * D + j0 + 4 * c]);  // row l as given
#pragma unroll
    for (int h = 0; h < 4; ++h) b.P[4 * c + h] = r4[h];
  }
#pragma unroll
  for (int ii = 0; ii < KB; ++ii) b.M[ii] = m0[(j0 + ii) * D + l];
  // A belief record: mean column l (rows J_w), covariance row l (columns J_w,
  // the diagonal folded in); record 0 is the initial belief as given.
  auto store = [&](float* mdst, float* cdst) __attribute__((always_inline)) {
#pragma unroll
    for (int ii = 0; ii < KB; ++ii) mdst[(j0 + ii) * D + l] = b.M[ii];
#pragma unroll
    for (int c = 0; c < KB / 4; ++c) {
      v4f r4;
#pragma unroll
      for (int h = 0; h < 4; ++h) r4[h] = (j0 + 4 * c + h == l) ? b.P[4 * c + h] + b.pd : b.P[4 * c + h];
      *reinterpret_cast<v4f*>(&cdst[l * D + j0 + 4 * c]) = r4;
    }
  };
  store(bm, bc);

  Prefetch<NT, FIXED> pf;
  if (T > 0) {
    pf.fetch(sp, 0, T, tid);
    pf.put(stage[0], tid);
  }
  __syncthreads();
  if (T > kBlk) pf.fetch(sp, kBlk, T, tid);
  float ypart = 0.f;  // the wave's partial of y of the previous token
  int64_t rec = 1, next_rec = a.chunk;
  for (int t = 0; t < T; ++t) {
    if (t == next_rec) {
      store(bm + rec * D * D, bc + rec * D * D);
      ++rec;
      next_rec += a.chunk;
    }
    const int tt = t % kBlk, blk = t / kBlk;
    TokG<KB> x;
    read_tok<KB, FIXED, false, true>(x, stage[blk & 1], tt, l, j0);
    v4f* xs = xz[t & 1];
    const v2f pz = predict_part(b, x);
    xs[w * kWave + l] = v4f{pz[0], pz[1], ypart, 0.f};
    const bool block_end = tt == kBlk - 1 && t + 1 < T;
    if (block_end) pf.put(stage[(blk + 1) & 1], tid);
    __syncthreads();
    float zs[W], es[W], ys[W];
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const v4f v = xs[i * kWave + l];
      zs[i] = v[0];
      es[i] = v[1];
      ys[i] = v[2];
    }
    if (block_end && t + 1 + kBlk < T) pf.fetch(sp, t + 1 + kBlk, T, tid);
    if (w == 0 && t > 0) yp[(t - 1) * D + l] = tree<W>(ys);
    const PredG o = predict_done<W>(b, x, zs, es, a.floor);
    update_g(b, x, o, l, j0, t == 0 ? c0 + l : nullptr);
    float ay[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ii = 0; ii < KB; ++ii) ay[ii & 3] = fmaf(b.M[ii], x.qJ[ii], ay[ii & 3]);
    ypart = (ay[0] + ay[1]) + (ay[2] + ay[3]);
  }
  if (T > 0) {
    v4f* xs = xz[T & 1];
    xs[w * kWave + l] = v4f{0.f, 0.f, ypart, 0.f};
    __syncthreads();
    float ys[W];
#pragma unroll
    for (int i = 0; i < W; ++i) ys[i] = xs[i * kWave + l][2];
    if (w == 0) yp[(T - 1) * D + l] = tree<W>(ys);
  }
  store(a.mT + n * D * D, a.cT + n * D * D);
  if (T > 0) store(bm + a.nb * D * D, bc + a.nb * D * D);
}

// Backward at checkpoint interval kBlk: each chunk is replayed once from its
// record with the belief blocks and intermediates of every token kept in
// registers, then reversed token by token (the reverse of
// persistent_bayes_chunked.cu:303-343 in the conventions of the one-wave
// kernel above: symmetrized gu k^T adjoint, first-token mirror correction).
// Barriers per token: one in the replay, two in the reverse.
template <int W, bool FIXED, bool DYN>
__global__ __launch_bounds__(W * kWave) __attribute__((amdgpu_waves_per_eu(W / 4, W / 4)))
void backward_group_kernel(BwdArgs a) {
  constexpr int KB = D / W, NT = W * kWave, G = kWave / KB;
  __shared__ v2f xz[2][W * kWave];
  __shared__ v2f xb[W * kWave], xc[W * kWave];
  __shared__ float ra[D], rkm[D], rdm[D];
  __shared__ __attribute__((aligned(16))) float tiles[W * kWave * KB];
  __shared__ __attribute__((aligned(16))) float stage[2][kStage];
  const int tid = static_cast<int>(threadIdx.x), w = wave_index(), l = tid & (kWave - 1), j0 = KB * w;
  float* tile = tiles + w * kWave * KB;
  const int64_t n = blockIdx.x;
  const int T = static_cast<int>(a.t);
  const int64_t nbp = a.nb + 1;
  const float* bm = a.bm + n * nbp * D * D;
  const float* bc = a.bc + n * nbp * D * D;
  const float* c0 = a.c0 + n * D * D;
  const Streams sp{a.k + n * T * D, a.v + n * T * D, a.q + n * T * D, a.gy + n * T * D,
                   FIXED ? nullptr : a.d + n * T * D, FIXED ? nullptr : a.p + n * T, FIXED ? nullptr : a.r + n * T};
  float* gkp = a.gk + n * T * D;
  float* gqp = a.gq + n * T * D;
  float* gvp = a.gv + n * T * D;
  float* gdp = a.gd ? a.gd + n * T * D : nullptr;
  float* gpp = a.gp ? a.gp + n * T : nullptr;
  float* grp = a.gr ? a.gr + n * T : nullptr;

  // Carried adjoints: S = sym(dL/dP) (row l, columns J_w; Sd the diagonal
  // part that pairs with pd), gM = dL/dM (column l, rows J_w).
  float S[KB], gM[KB], Sd = 0.f;
  if (a.gmf) {
    const float* gmf = a.gmf + n * D * D;
#pragma unroll
    for (int ii = 0; ii < KB; ++ii) gM[ii] = gmf[(j0 + ii) * D + l];
  } else {
#pragma unroll
    for (int ii = 0; ii < KB; ++ii) gM[ii] = 0.f;
  }
  if (a.gcf) {
    const float* gcf = a.gcf + n * D * D;
#pragma unroll
    for (int jj = 0; jj < KB; ++jj) {
      const int j = j0 + jj;
      S[jj] = 0.5f * (gcf[l * D + j] + gcf[j * D + l]);
    }
    Sd = 0.5f * (gcf[l * D + l] + gcf[l * D + l]);
  } else {
#pragma unroll
    for (int jj = 0; jj < KB; ++jj) S[jj] = 0.f;
  }

  const int nb = static_cast<int>(a.nb);
  // Stage of the last chunk; each chunk c > 0 issues the loads of chunk
  // c - 1 after its first barrier (the other stage buffer is free then) and
  // publishes them at its last.
  float pr = 0.f;
  if (nb > 0) {
    stage_dma<NT, FIXED>(sp, stage[(nb - 1) & 1], (nb - 1) * kBlk, T, tid);
    if (!FIXED && tid < 2 * kBlk) stage[(nb - 1) & 1][kSP + tid] = dma_pr(sp, (nb - 1) * kBlk, T, tid);
    r4::vm_wait<0>();
  }
  __syncthreads();
  int par = 0;
  for (int c = nb - 1; c >= 0; --c) {
    bool dma_pending = c > 0;
    const int t0 = c * kBlk;
    const int len = (T - t0) < kBlk ? (T - t0) : kBlk;
    const float* st = stage[c & 1];
    // One pass: replay tokens [0, min(len, HI)) from the chunk's record,
    // keeping the beliefs and intermediates of tokens [LO, HI), then reverse
    // those tokens.
    auto pass = [&](auto lo_c, auto hi_c) __attribute__((always_inline)) {
      constexpr int LO = decltype(lo_c)::value, HI = decltype(hi_c)::value, NH = HI - LO;
      BelG<KB> hb[NH];
      PredG ho[NH];
      {
        BelG<KB> b;
        const float* cm = bm + static_cast<int64_t>(c) * D * D;
        const float* cc = bc + static_cast<int64_t>(c) * D * D;
#pragma unroll
        for (int q4 = 0; q4 < KB / 4; ++q4) {
          const v4f r4 = *reinterpret_cast<const v4f*>(&cc[l * D + j0 + 4 * q4]);
#pragma unroll
          for (int h = 0; h < 4; ++h) b.P[4 * q4 + h] = r4[h];
        }
#pragma unroll
        for (int ii = 0; ii < KB; ++ii) b.M[ii] = cm[(j0 + ii) * D + l];
        b.pd = 0.f;
#pragma unroll
        for (int tt = 0; tt < HI; ++tt) {
          if (tt < len) {
            TokG<KB> x;
            read_tok<KB, FIXED, false>(x, st, tt, l, j0);
            if (tt >= LO) hb[tt >= LO ? tt - LO : 0] = b;
            v2f* xs = xz[par];
            par ^= 1;
            xs[w * kWave + l] = predict_part(b, x);
            __syncthreads();
            if (tt == 0 && dma_pending) {
              stage_dma<NT, FIXED>(sp, stage[(c - 1) & 1], (c - 1) * kBlk, T, tid);
              if (!FIXED && tid < 2 * kBlk) pr = dma_pr(sp, (c - 1) * kBlk, T, tid);
              dma_pending = false;
            }
            float zs[W], es[W];
#pragma unroll
            for (int i = 0; i < W; ++i) {
              const v2f v = xs[i * kWave + l];
              zs[i] = v[0];
              es[i] = v[1];
            }
            const PredG o = predict_done<W>(b, x, zs, es, a.floor);
            if (tt >= LO) ho[tt >= LO ? tt - LO : 0] = o;
            if (tt + 1 < len && tt + 1 < HI) update_g(b, x, o, l, j0, (c == 0 && tt == 0) ? c0 + l : nullptr);
          }
        }
      }
#pragma unroll
      for (int tt = HI - 1; tt >= LO; --tt) {
        if (tt < len) {
          const BelG<KB>& hbt = hb[tt - LO];
          const PredG& o = ho[tt - LO];
          const int t = t0 + tt;
          TokG<KB> x;
          read_tok<KB, FIXED, true>(x, st, tt, l, j0);
          float uJ[KB], dM[KB];
#pragma unroll
          for (int jj = 0; jj < KB; ++jj) {
            uJ[jj] = lane_value(o.u, j0 + jj);
            dM[jj] = x.dJ[jj] * hbt.M[jj];
          }
          // Phase 1: gM += q gy^T; partials of gM^T u and S u; row sums of
          // M_new gy (dL/dq) and gM e.
          float am[4] = {0.f, 0.f, 0.f, 0.f}, aw[4] = {0.f, 0.f, 0.f, 0.f};
          float vq[KB], va[KB];
          const float be = o.beta * o.e;
#pragma unroll
          for (int ii = 0; ii < KB; ++ii) {
            gM[ii] = fmaf(x.qJ[ii], x.gy, gM[ii]);
            am[ii & 3] = fmaf(gM[ii], uJ[ii], am[ii & 3]);
            aw[ii & 3] = fmaf(S[ii], uJ[ii], aw[ii & 3]);
            vq[ii] = fmaf(uJ[ii], be, dM[ii]) * x.gy;
            va[ii] = gM[ii] * o.e;
          }
          {
            const float rq = lane_rowsum<KB>(tile, l, vq);
            if (l % G == 0) gqp[t * D + j0 + l / G] = rq;
            const float r_a = lane_rowsum<KB>(tile, l, va);
            if (l % G == 0) ra[j0 + l / G] = r_a;
          }
          xb[w * kWave + l] = v2f{(am[0] + am[1]) + (am[2] + am[3]), (aw[0] + aw[1]) + (aw[2] + aw[3])};
          __syncthreads();
          // Phase 2: ge, gs, gu; row sums of (d M) ge and (gM - k ge^T) M;
          // partials of P' gu and of the decay's covariance term.  gu enters
          // halved (hg = gu / 2, exact), which gives the symmetrized outer
          // product sym(gu k^T) without a further rounding.
          float gms[W], ws[W];
#pragma unroll
          for (int i = 0; i < W; ++i) {
            const v2f v = xb[i * kWave + l];
            gms[i] = v[0];
            ws[i] = v[1];
          }
          const float gmu = tree<W>(gms), wl = tree<W>(ws);
          const float a_l = ra[l];
          const float ge = o.beta * gmu;
          const float z = wave_total(fmaf(o.e, gmu, -(o.u * wl)));
          const float gs = o.clamped ? 0.f : -z * o.beta * o.beta;
          const float gu = fmaf(o.beta, fmaf(-2.f, wl, a_l), gs * x.k);
          const float hg = 0.5f * gu;
          float vk[KB], vd[KB];
#pragma unroll
          for (int ii = 0; ii < KB; ++ii) {
            vk[ii] = dM[ii] * ge;
            const float g = fmaf(-x.kJ[ii], ge, gM[ii]);
            vd[ii] = g * hbt.M[ii];
            gM[ii] = g * x.dJ[ii];
          }
          {
            const float r_k = lane_rowsum<KB>(tile, l, vk);
            if (l % G == 0) rkm[j0 + l / G] = r_k;
            if constexpr (DYN) {
              const float r_d = lane_rowsum<KB>(tile, l, vd);
              if (l % G == 0) rdm[j0 + l / G] = r_d;
            }
          }
          float ap[4] = {0.f, 0.f, 0.f, 0.f}, gdc = 0.f;
          const bool first = t == 0;
#pragma unroll
          for (int jj = 0; jj < KB; ++jj) {
            const int j = j0 + jj;
            const float hj = lane_value(hg, j);
            const float dd = mul_rn(x.d, x.dJ[jj]);
            ap[jj & 3] = fmaf(hbt.P[jj] * dd, hj, ap[jj & 3]);
            if (first && j < l) ap[jj & 3] = fmaf((c0[j * D + l] - hbt.P[jj]) * dd, hj, ap[jj & 3]);
            const float h = add_rn(S[jj], add_rn(mul_rn(hg, x.kJ[jj]), mul_rn(hj, x.k)));
            if constexpr (DYN) gdc = fmaf(h * hbt.P[jj], x.dJ[jj], gdc);
            S[jj] = h * dd;
          }
          const float hd = add_rn(Sd, add_rn(mul_rn(hg, x.k), mul_rn(hg, x.k)));
          Sd = hd * mul_rn(x.d, x.d);
          xc[w * kWave + l] = v2f{(ap[0] + ap[1]) + (ap[2] + ap[3]), gdc};
          if (tt == 0 && c > 0) {  // publish the next chunk's stage
            if (!FIXED && tid < 2 * kBlk) stage[(c - 1) & 1][kSP + tid] = pr;
            r4::vm_wait<0>();
          }
          __syncthreads();
          // Phase 3: dL/dk, dL/dd, dL/dp, dL/dr of the token (P' gu = 2 P' hg).
          float pgs[W], gds[W];
#pragma unroll
          for (int i = 0; i < W; ++i) {
            const v2f v = xc[i * kWave + l];
            pgs[i] = v[0];
            gds[i] = v[1];
          }
          const float pgu = 2.f * tree<W>(pgs);
          const float gk = -rkm[l] + fmaf(gs, o.u, fmaf(fmaf(hbt.pd, mul_rn(x.d, x.d), x.p), gu, pgu));
          if (w == 0) {
            gkp[t * D + l] = gk;
            gvp[t * D + l] = ge;
          }
          if constexpr (DYN) {
            const float gdl = fmaf(hd * hbt.pd, x.d, tree<W>(gds));
            const float gd = fmaf(2.f, gdl, rdm[l]);
            const float gp = wave_total(hd);
            if (w == 0) {
              if (gdp) gdp[t * D + l] = gd;
              if (l == 0) {
                if (gpp) gpp[t] = gp;
                if (grp) grp[t] = gs;
              }
            }
          } else if (w == 0) {
            if (gdp) gdp[t * D + l] = 0.f;
            if (l == 0) {
              if (gpp) gpp[t] = 0.f;
              if (grp) grp[t] = 0.f;
            }
          }
        }
      }
    };
    pass(std::integral_constant<int, 0>{}, std::integral_constant<int, kBlk>{});
  }
  if (a.gm0) {
#pragma unroll
    for (int ii = 0; ii < KB; ++ii) a.gm0[n * D * D + (j0 + ii) * D + l] = gM[ii];
  }
  if (a.gc0) {
#pragma unroll
    for (int jj = 0; jj < KB; ++jj) a.gc0[n * D * D + (j0 + jj) * D + l] = S[jj];
  }
}

}  // namespace d64

hipError_t launch_forward_d64(bool fixed, const FwdArgs& a, hipStream_t stream) {
  if (a.n == 0) return hipSuccess;
  constexpr int W = d64::kForwardWaves;
  const dim3 grid(static_cast<unsigned>(a.n)), block(W * kWave);
  if (fixed) hipLaunchKernelGGL((d64::forward_group_kernel<W, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((d64::forward_group_kernel<W, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_backward_d64(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  if (a.n == 0) return hipSuccess;
  if (a.chunk == d64::kBlk) {
    constexpr int W = d64::kBackwardWaves;
    const dim3 grid(static_cast<unsigned>(a.n)), block(W * kWave);
    if (fixed) hipLaunchKernelGGL((d64::backward_group_kernel<W, true, false>), grid, block, 0, stream, a);
    else if (dyn) hipLaunchKernelGGL((d64::backward_group_kernel<W, false, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((d64::backward_group_kernel<W, false, false>), grid, block, 0, stream, a);
    return hipGetLastError();
  }
  const dim3 grid(static_cast<unsigned>(a.n)), block(kWave);
  if (fixed) hipLaunchKernelGGL((d64::backward_kernel<true, false>), grid, block, 0, stream, a);
  else if (dyn) hipLaunchKernelGGL((d64::backward_kernel<false, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((d64::backward_kernel<false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace bssm
