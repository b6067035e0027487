// gfx950 checkpoint-replay backward for D = 8, M = 8
// (bayes_ssm/persistent_bayes_chunked_d8.cu:358-419 is the reference reverse
// for this shape; the per-token equations are those of bssm_step.h and the
// reverse conventions those of the D = 4 kernels in bssm_rot4.h).
//
// A wave holds 8 sequences; lane l = 8 s + g owns covariance row g and value
// column g of sequence s.  Every per-index quantity a lane holds is stored
// in XOR order: slot m holds index g ^ m, so
//   P[m] = P[g][g ^ m]     Mv[m] = M[g ^ m][g]     kx[m] = k[g ^ m]
// and the 8-lane exchanges are butterflies of single DPP moves (xor 1, xor 2
// and the half-row mirror, which is xor 7 inside each 8-lane group):
//   all-gather (slot m <- lane g ^ m's own value):     7 moves
//   reduce-scatter (per-index partials -> own total):  7 fused adds
//   all-reduce (per-sequence scalars):                 3 fused adds, the same
//                                                     bits in all 8 lanes
// Entry (g, j) of the covariance and its mirror (j, g) are computed by two
// lanes from commutative products only, so the covariance stays bitwise
// symmetric.
//
// The backward replays each 8-token checkpoint chunk on chip (the belief
// before each token and the step's u_g, s, e_g kept in registers), then
// reverses it; the next chunk's inputs and checkpoint record arrive by
// LDS-DMA meanwhile (ring of 2 slots).  LDS layouts of a slot (floats):
//   k, d, q, v, gy: token-major [8 t][8 s][8] (lane (s, g) reads index g ^ m
//     of token t at (8 t + s) * 8 + (g ^ m): 64 distinct banks per read);
//   p, r: [8 s][8 t] (+ padding);  checkpoint records: mean, covariance
//     [8 s][64].
// Gradients overwrite their inputs in place and leave through the same maps.

#include "bssm_rot4.h"
#include "bssm_step.h"

namespace bssm {
namespace d8 {

using r4::dma16;
using r4::kOob;
using r4::lds_wait;
using r4::make_rsrc;
using r4::Rsrc;
using r4::st128;
using r4::vm_wait;

constexpr int SPW = 8;      // sequences per wave
constexpr int kChunk = 8;   // checkpoint chunk, tokens
constexpr bool kNt = r4::kNtLoad;
constexpr int kNtSt = r4::kNtStore;

// p and r take 256 floats each: their DMA instruction's lanes past 16 carry
// no piece and fill the padding after the 64 used floats with zeros.
struct Slot {
  static constexpr int K = 0, D = 512, Q = 1024, V = 1536, GY = 2048, P = 2560, R = 2816, CKM = 3072, CKC = 3584,
                       SIZE = 4096;
};

// ------------------------------------------------------ 8-lane exchanges
// x[m] <- the own value of lane g ^ m of the group (x[0] = own).
__device__ __forceinline__ void gather8(float own, float (&x)[8]) {
  x[0] = own;
  x[1] = dpp<kXor1>(x[0]);
  x[2] = dpp<kXor2>(x[0]);
  x[3] = dpp<kXor2>(x[1]);
  x[7] = dpp<kHalfMirror>(x[0]);
  x[6] = dpp<kHalfMirror>(x[1]);
  x[5] = dpp<kHalfMirror>(x[2]);
  x[4] = dpp<kHalfMirror>(x[3]);
}
// Group total for the lane's own index g of per-slot partials (x[m]: the
// lane's partial for index g ^ m): recursive halving over xor 7, 2, 1.
__device__ __forceinline__ float reduce_scatter8(const float (&x)[8]) {
  float y[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) y[m] = x[m] + dpp<kHalfMirror>(x[m ^ 7]);
  const float z0 = y[0] + dpp<kXor2>(y[2]);
  const float z1 = y[1] + dpp<kXor2>(y[3]);
  return z0 + dpp<kXor1>(z1);
}
// Sum over the group; the same bits in all 8 lanes (each stage adds the two
// halves of a symmetric pairing).
__device__ __forceinline__ float all_reduce8(float x) {
  x += dpp<kXor1>(x);
  x += dpp<kXor2>(x);
  return x + dpp<kHalfMirror>(x);
}

// ------------------------------------------------------------ per token
struct Bel {
  float P[8];   // P[g][g ^ m]
  float Mv[8];  // M[g ^ m][g]
};
struct Tok {
  float kx[8], dx[8];
  float v, p, r;
};
struct RevTok {
  float kx[8], dx[8], qx[8];
  float gy, p;
};
// Everything the reverse of a token needs that is not a token input: the
// belief before it and the step's u_g, unclamped s and own innovation.
struct Hist {
  float Pp[8], Mp[8];
  float ug, s, e;
};

// One token of the recurrence (bayesian_layer.py:207-251): u = P' k with
// P' = d P d + p I, s = r + k.u, beta = 1 / max(s, floor), e = v - (d M)^T k,
// M <- d M + u (beta e)^T, P <- P' - beta u u^T.
__device__ __forceinline__ void step(Bel& b, const Tok& in, float floor, Hist& h) {
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    h.Pp[m] = b.P[m];
    h.Mp[m] = b.Mv[m];
  }
  float wk[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) wk[m] = in.dx[m] * in.kx[m];
  float z = b.P[0] * wk[0];
#pragma unroll
  for (int m = 1; m < 8; ++m) z = fmaf(b.P[m], wk[m], z);
  const float ug = fmaf(in.dx[0], z, in.p * in.kx[0]);
  const float s = all_reduce8(in.kx[0] * ug) + in.r;
  const float beta = fast_rcp(fmaxf(s, floor));
  float ux[8];
  gather8(ug, ux);
  float e = in.v;
#pragma unroll
  for (int m = 0; m < 8; ++m) e = fmaf(-b.Mv[m], wk[m], e);
  const float be = beta * e;
#pragma unroll
  for (int m = 0; m < 8; ++m) b.Mv[m] = fmaf(ux[m], be, in.dx[m] * b.Mv[m]);
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    float dp = (in.dx[0] * in.dx[m]) * b.P[m];
    if (m == 0) dp += in.p;
    b.P[m] = fmaf(-beta, ug * ux[m], dp);
  }
  h.ug = ug;
  h.s = s;
  h.e = e;
}

struct RevOut {
  float gk, gq, gd, gv, gp, gr, gu;
};

// Reverse of one token (the D = 4 reverse_step of bssm_rot4.h with one value
// column per lane).  Carried adjoints: gM = dL/dM (own column) and S =
// sym(dL/dP) (own row), updated in place to their values before the token;
// Mn is the mean after the token (own column).
template <bool DYN>
__device__ __forceinline__ void reverse_step(const RevTok& in, const Hist& h, const float (&Mn)[8],
                                             float (&gM)[8], float (&S)[8], float floor, RevOut& o) {
  const float beta = fast_rcp(fmaxf(h.s, floor));
  float ux[8];
  gather8(h.ug, ux);
#pragma unroll
  for (int m = 0; m < 8; ++m) gM[m] = fmaf(in.qx[m], in.gy, gM[m]);
  float ge = gM[0] * ux[0];
#pragma unroll
  for (int m = 1; m < 8; ++m) ge = fmaf(gM[m], ux[m], ge);
  ge *= beta;
  o.gv = ge;
  float av[8], Av[8], Cv[8], Bv[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    av[m] = gM[m] * h.e;
    Av[m] = h.Mp[m] * ge;
    Cv[m] = Mn[m] * in.gy;
    const float gb = fmaf(-in.kx[m], ge, gM[m]);
    gM[m] = gb * in.dx[m];
    Bv[m] = DYN ? gb * h.Mp[m] : 0.f;
  }
  const float a_g = reduce_scatter8(av);
  const float A_g = reduce_scatter8(Av);
  o.gq = reduce_scatter8(Cv);
  float w = S[0] * ux[0];
#pragma unroll
  for (int m = 1; m < 8; ++m) w = fmaf(S[m], ux[m], w);
  const float z = all_reduce8(h.ug * (a_g - w));
  const float gs = (h.s > floor) ? -z * beta * beta : 0.f;
  const float gu = fmaf(beta, fmaf(-2.f, w, a_g), gs * in.kx[0]);
  float gux[8];
  gather8(gu, gux);
  float dd[8], gk = fmaf(-in.dx[0], A_g, gs * h.ug);
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    dd[m] = in.dx[0] * in.dx[m];
    float pb = dd[m] * h.Pp[m];
    if (m == 0) pb += in.p;
    gk = fmaf(pb, gux[m], gk);
  }
  o.gk = gk;
  const float hg = 0.5f * gu, hk = 0.5f * in.kx[0];
  float gd = 0.f;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const float hs = fmaf(hg, in.kx[m], fmaf(gux[m], hk, S[m]));
    if (DYN) gd = fmaf(hs * in.dx[m], h.Pp[m], gd);
    if (m == 0) o.gp = DYN ? all_reduce8(hs) : 0.f;
    S[m] = hs * dd[m];
  }
  o.gd = DYN ? fmaf(2.f, gd, reduce_scatter8(Bv)) : 0.f;
  o.gr = DYN ? gs : 0.f;
  o.gu = gu;
}

// ------------------------------------------------------------ backward
template <bool FIXED, bool DYN>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(1, 1))) void backward_kernel(BwdArgs a) {
  __shared__ float ta[Slot::SIZE], tb[Slot::SIZE];
  const int lane = threadIdx.x;
  const int g = lane & 7, s = lane >> 3;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t T = a.t;
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  const uint32_t row8 = static_cast<uint32_t>(T) * 32u, row1 = static_cast<uint32_t>(T) * 4u;
  const Rsrc rk = make_rsrc(a.k + n0 * T * 8, valid * row8);
  const Rsrc rq = make_rsrc(a.q + n0 * T * 8, valid * row8);
  const Rsrc rv = make_rsrc(a.v + n0 * T * 8, valid * row8);
  const Rsrc rgy = make_rsrc(a.gy + n0 * T * 8, valid * row8);
  const Rsrc rd = make_rsrc(FIXED ? a.k : a.d + n0 * T * 8, valid * row8);
  const Rsrc rp = make_rsrc(FIXED ? a.k : a.p + n0 * T, valid * row1);
  const Rsrc rr = make_rsrc(FIXED ? a.k : a.r + n0 * T, valid * row1);
  const Rsrc rgk = make_rsrc(a.gk + n0 * T * 8, valid * row8);
  const Rsrc rgq = make_rsrc(a.gq + n0 * T * 8, valid * row8);
  const Rsrc rgv = make_rsrc(a.gv + n0 * T * 8, valid * row8);
  const Rsrc rgd = make_rsrc(a.gd ? a.gd + n0 * T * 8 : a.gk, a.gd ? valid * row8 : 0u);
  const Rsrc rgp = make_rsrc(a.gp ? a.gp + n0 * T : a.gk, a.gp ? valid * row1 : 0u);
  const Rsrc rgr = make_rsrc(a.gr ? a.gr + n0 * T : a.gk, a.gr ? valid * row1 : 0u);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 64, valid * nbp * 256u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 64, valid * nbp * 256u);

  // DMA / store maps (byte offsets relative to the chunk's first token).
  // 8-value streams, instruction j < 2: token 4 j + (l >> 4), sequence
  // (l >> 1) & 7, half l & 1 -> LDS float 256 j + 4 l ([t][s][8]).
  uint32_t o8[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    o8[j] = static_cast<uint32_t>((lane >> 1) & 7) * row8 + static_cast<uint32_t>(4 * j + (lane >> 4)) * 32u +
            static_cast<uint32_t>(lane & 1) * 16u;
  // p, r: lanes < 16: sequence l >> 1, tokens 4 (l & 1) .. + 3 -> LDS float 4 l ([s][8]).
  const uint32_t o1 = lane < 16 ? static_cast<uint32_t>(lane >> 1) * row1 + static_cast<uint32_t>(lane & 1) * 16u
                                : kOob;
  // Checkpoint records, instruction j < 2: sequence 4 j + (l >> 4), piece l & 15 -> LDS float 256 j + 4 l.
  uint32_t orec[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    orec[j] = static_cast<uint32_t>(4 * j + (lane >> 4)) * (nbp * 256u) + static_cast<uint32_t>(lane & 15) * 16u;

  // Per-lane LDS float offsets of the XOR-ordered reads of a token row
  // (token 0; token t adds 64 t).
  int ix[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) ix[m] = s * 8 + (g ^ m);

  // Carried adjoints from the final-state gradients (null = zero).
  float gM[8], S[8];
  {
    const bool has_m = a.gmf != nullptr, has_c = a.gcf != nullptr;
    const Rsrc rgm = make_rsrc(has_m ? a.gmf + n0 * 64 : a.m0, has_m ? valid * 256u : 0u);
    const Rsrc rgc = make_rsrc(has_c ? a.gcf + n0 * 64 : a.m0, has_c ? valid * 256u : 0u);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int j = g ^ m;
      gM[m] = r4::ld32(rgm, static_cast<uint32_t>(s * 256 + j * 32 + g * 4), 0);
      S[m] = 0.5f * (r4::ld32(rgc, static_cast<uint32_t>(s * 256 + g * 32 + j * 4), 0) +
                     r4::ld32(rgc, static_cast<uint32_t>(s * 256 + j * 32 + g * 4), 0));
    }
  }
  float first_gu = 0.f;

  auto issue = [&](float* tl, int64_t c) __attribute__((always_inline)) {
    const int64_t t0 = c * kChunk;
    const uint32_t s8 = static_cast<uint32_t>(t0) * 32u, s1 = static_cast<uint32_t>(t0) * 4u;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      dma16<kNt>(rk, tl + Slot::K + 256 * j, o8[j] + s8);
      dma16<kNt>(rq, tl + Slot::Q + 256 * j, o8[j] + s8);
      if constexpr (!FIXED) dma16<kNt>(rd, tl + Slot::D + 256 * j, o8[j] + s8);
      dma16<kNt>(rv, tl + Slot::V + 256 * j, o8[j] + s8);
      dma16<kNt>(rgy, tl + Slot::GY + 256 * j, o8[j] + s8);
    }
    if constexpr (!FIXED) {
      dma16(rp, tl + Slot::P, o1 == kOob ? kOob : o1 + s1);
      dma16(rr, tl + Slot::R, o1 == kOob ? kOob : o1 + s1);
    }
    const uint32_t cr = static_cast<uint32_t>(c) * 256u;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      dma16<kNt>(rbm, tl + Slot::CKM + 256 * j, orec[j] + cr);
      dma16<kNt>(rbc, tl + Slot::CKC + 256 * j, orec[j] + cr);
    }
  };
  auto store_grads = [&](const float* tl, int64_t c) __attribute__((always_inline)) {
    const int64_t t0 = c * kChunk;
    const uint32_t s8 = static_cast<uint32_t>(t0) * 32u, s1 = static_cast<uint32_t>(t0) * 4u;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = 256 * j + 4 * lane;
      st128<kNtSt>(rgk, *reinterpret_cast<const v4f*>(&tl[Slot::K + e]), o8[j], s8);
      st128<kNtSt>(rgq, *reinterpret_cast<const v4f*>(&tl[Slot::Q + e]), o8[j], s8);
      if (a.gd) st128<kNtSt>(rgd, *reinterpret_cast<const v4f*>(&tl[Slot::D + e]), o8[j], s8);
      st128<kNtSt>(rgv, *reinterpret_cast<const v4f*>(&tl[Slot::V + e]), o8[j], s8);
    }
    if (a.gp) st128(rgp, *reinterpret_cast<const v4f*>(&tl[Slot::P + 4 * (lane & 15)]), o1, s1);
    if (a.gr) st128(rgr, *reinterpret_cast<const v4f*>(&tl[Slot::R + 4 * (lane & 15)]), o1, s1);
  };

  auto read_tok = [&](const float* tl, int tt, Tok& x) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      x.kx[m] = tl[Slot::K + 64 * tt + ix[m]];
      x.dx[m] = FIXED ? kFixedDecay : tl[Slot::D + 64 * tt + ix[m]];
    }
    x.v = tl[Slot::V + 64 * tt + ix[0]];
    x.p = FIXED ? kFixedProcess : tl[Slot::P + 8 * s + tt];
    x.r = FIXED ? kFixedObservation : tl[Slot::R + 8 * s + tt];
  };
  auto read_rev = [&](const float* tl, int tt, RevTok& x) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      x.kx[m] = tl[Slot::K + 64 * tt + ix[m]];
      x.dx[m] = FIXED ? kFixedDecay : tl[Slot::D + 64 * tt + ix[m]];
      x.qx[m] = tl[Slot::Q + 64 * tt + ix[m]];
    }
    x.gy = tl[Slot::GY + 64 * tt + ix[0]];
    x.p = FIXED ? kFixedProcess : tl[Slot::P + 8 * s + tt];
  };
  // Replay of a whole chunk from its checkpoint, then its reverse; the
  // gradients overwrite the chunk's inputs.  Each token's LDS reads are
  // issued one token ahead.
  auto process = [&](float* tl, int64_t c) __attribute__((always_inline)) {
    Bel b;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      b.P[m] = tl[Slot::CKC + s * 64 + g * 8 + (g ^ m)];
      b.Mv[m] = tl[Slot::CKM + s * 64 + (g ^ m) * 8 + g];
    }
    Hist h[kChunk];
    Tok x[kChunk];
    RevTok rx[kChunk];
    read_tok(tl, 0, x[0]);
#pragma unroll
    for (int tt = 0; tt < kChunk; ++tt) {
      if (tt + 1 < kChunk) read_tok(tl, tt + 1, x[tt + 1]);
      else read_rev(tl, kChunk - 1, rx[kChunk - 1]);
      __builtin_amdgcn_sched_barrier(0);
      step(b, x[tt], a.floor, h[tt]);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int tt = kChunk - 1; tt >= 0; --tt) {
      if (tt > 0) read_rev(tl, tt - 1, rx[tt - 1]);
      __builtin_amdgcn_sched_barrier(0);
      RevOut o;
      reverse_step<DYN>(rx[tt], h[tt], tt + 1 < kChunk ? h[tt + 1 < kChunk ? tt + 1 : tt].Mp : b.Mv, gM, S,
                        a.floor, o);
      if (tt == 0) first_gu = o.gu;
      tl[Slot::K + 64 * tt + ix[0]] = o.gk;
      tl[Slot::Q + 64 * tt + ix[0]] = o.gq;
      tl[Slot::D + 64 * tt + ix[0]] = o.gd;
      tl[Slot::V + 64 * tt + ix[0]] = o.gv;
      if (g == 0) {
        tl[Slot::P + 8 * s + tt] = o.gp;
        tl[Slot::R + 8 * s + tt] = o.gr;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Chunk c = nb - 1 - i in slot i % 2: at its start the loads issued a
  // whole chunk earlier are awaited, the gradients of chunk c + 1 leave the
  // other slot, which then receives chunk c - 1.
  const int64_t nb = a.nb;
  auto run_chunk = [&](float* cur, float* other, int64_t c) __attribute__((always_inline)) {
    vm_wait<0>();
    if (c + 1 < nb) store_grads(other, c + 1);
    if (c > 0) {
      lds_wait();
      issue(other, c - 1);
    }
    process(cur, c);
  };
  if (nb > 0) issue(ta, nb - 1);
  for (int64_t i = 0; i < nb; i += 2) {
    run_chunk(ta, tb, nb - 1 - i);
    if (i + 1 < nb) run_chunk(tb, ta, nb - 2 - i);
  }
  float* last = (nb - 1) % 2 == 0 ? ta : tb;  // slot of chunk 0
  lds_wait();
  if (nb > 0) store_grads(last, 0);

  // Adjoints of the initial mean and covariance.  The covariance one is the
  // full (asymmetric) derivative (S_in + gu k^T) * d d^T of the first token
  // (persistent_bayes_chunked_d8.cu:396-405), recovered from the carried
  // S_out = (S_in + sym(gu k^T)) * d d^T.  Token 0's k and d in its slot
  // were overwritten by their gradients, so they are read back from the
  // caller's tensors.
  if (a.gm0) {
    const Rsrc rgm0 = make_rsrc(a.gm0 + n0 * 64, valid * 256u);
#pragma unroll
    for (int m = 0; m < 8; ++m) r4::st32(rgm0, gM[m], static_cast<uint32_t>(s * 256 + (g ^ m) * 32 + g * 4), 0);
  }
  if (a.gc0) {
    float kx[8], dx[8], gux[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const uint32_t off = static_cast<uint32_t>(s) * row8 + static_cast<uint32_t>(g ^ m) * 4u;
      kx[m] = r4::ld32(rk, off, 0);
      dx[m] = FIXED ? kFixedDecay : r4::ld32(rd, off, 0);
    }
    gather8(first_gu, gux);
    const Rsrc rgc0 = make_rsrc(a.gc0 + n0 * 64, valid * 256u);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const float asym = 0.5f * fmaf(first_gu, kx[m], -gux[m] * kx[0]);
      r4::st32(rgc0, fmaf(asym, dx[0] * dx[m], S[m]), static_cast<uint32_t>(s * 256 + g * 32 + (g ^ m) * 4), 0);
    }
  }
}

// ------------------------------------------------------------- forward
// The backward's lane layout and step(), so the backward's replay rebuilds
// the forward's beliefs bit for bit.  16-token tiles are staged in
// registers (the next tile's loads are in flight while the current one is
// computed from LDS); every load instruction covers whole 512-byte row
// segments of two sequences, and the pieces are written to the token-major
// LDS layout [t][s][8] whose XOR-ordered per-token reads hit 64 distinct
// banks.  Readouts overwrite the consumed values in LDS and leave through
// the loads' map.  Checkpoint records at 8-token boundaries are staged
// through the spent half of the tile and leave as whole 16-byte pieces
// (cached: 8 us faster than with the nontemporal hint, and 80 us faster
// than 4-byte stores from the XOR-ordered registers); other records are
// stored entry by entry.
struct FwdSlot {
  static constexpr int K = 0, D = 1024, Q = 2048, V = 3072, P = 4096, R = 4224, SIZE = 4352;
};
constexpr int kFwdTile = 16;

// Register staging of one tile: 8-value streams, instruction I < 4: lane l
// -> sequence 2 I + (l >> 5), piece l & 31 (token (l & 31) >> 1, half l & 1);
// p, r: lanes < 32 -> sequence l >> 2, tokens 4 (l & 3) .. + 3.
struct FwdStage {
  v4f k[4], d[4], q[4], v[4], p, r;
};

template <bool FIXED>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(2))) void forward_kernel(FwdArgs a) {
  __shared__ float tile[FwdSlot::SIZE];
  const int lane = threadIdx.x;
  const int g = lane & 7, s = lane >> 3;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t T = a.t;
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  const uint32_t row8 = static_cast<uint32_t>(T) * 32u, row1 = static_cast<uint32_t>(T) * 4u;
  const Rsrc rk = make_rsrc(a.k + n0 * T * 8, valid * row8);
  const Rsrc rq = make_rsrc(a.q + n0 * T * 8, valid * row8);
  const Rsrc rv = make_rsrc(a.v + n0 * T * 8, valid * row8);
  const Rsrc ry = make_rsrc(a.y + n0 * T * 8, valid * row8);
  const Rsrc rd = make_rsrc(FIXED ? a.k : a.d + n0 * T * 8, FIXED ? 0u : valid * row8);
  const Rsrc rp = make_rsrc(FIXED ? a.k : a.p + n0 * T, FIXED ? 0u : valid * row1);
  const Rsrc rr = make_rsrc(FIXED ? a.k : a.r + n0 * T, FIXED ? 0u : valid * row1);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 64, valid * nbp * 256u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 64, valid * nbp * 256u);

  // Load / store map of the 8-value streams (byte offset inside the row
  // block, relative to the tile's first token; LDS float offset).
  const int c32 = lane & 31, tok8 = c32 >> 1;
  uint32_t o8[4];
  int l8[4];
#pragma unroll
  for (int I = 0; I < 4; ++I) {
    const int sq = 2 * I + (lane >> 5);
    o8[I] = static_cast<uint32_t>(sq) * row8 + static_cast<uint32_t>(c32) * 16u;
    l8[I] = 64 * tok8 + 8 * sq + 4 * (lane & 1);
  }
  const int tok1 = 4 * (lane & 3);
  const uint32_t o1 = lane < 32 ? static_cast<uint32_t>(lane >> 2) * row1 + static_cast<uint32_t>(lane & 3) * 16u
                                : kOob;

  // XOR-ordered LDS reads of a token row (token 0; token t adds 64 t).
  int ix[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) ix[m] = s * 8 + (g ^ m);

  // Belief of the lane: covariance row g and mean column g, XOR order.
  Bel b;
  {
    const Rsrc rm0 = make_rsrc(a.m0 + n0 * 64, valid * 256u);
    const Rsrc rc0 = make_rsrc(a.c0 + n0 * 64, valid * 256u);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      b.P[m] = r4::ld32(rc0, static_cast<uint32_t>(s * 256 + g * 32 + (g ^ m) * 4), 0);
      b.Mv[m] = r4::ld32(rm0, static_cast<uint32_t>(s * 256 + (g ^ m) * 32 + g * 4), 0);
    }
  }
  vm_wait<0>();
  const uint32_t rec_seq = static_cast<uint32_t>(s) * nbp * 256u;
  auto store_bel = [&](Rsrc rm, Rsrc rc, uint32_t base, uint32_t soff) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      r4::st32(rc, b.P[m], base + static_cast<uint32_t>(g * 32 + (g ^ m) * 4), soff);
      r4::st32(rm, b.Mv[m], base + static_cast<uint32_t>((g ^ m) * 32 + g * 4), soff);
    }
  };
  // Record c, entry by entry (records inside a tile's first half).
  auto store_ckpt = [&](uint32_t c) __attribute__((always_inline)) { store_bel(rbm, rbc, rec_seq, c * 256u); };
  // Record c through LDS: the belief is written over the spent first half
  // of the tile's K (means) and D (covariances) regions, each sequence's
  // 8 x 8 block with row r at position (r + s) % 8 (the XOR-ordered writes
  // of 64 lanes then hit 64 distinct banks), read back as 16-byte pieces
  // (instruction j < 2: lane l -> sequence 4 j + (l >> 4), piece l & 15)
  // and stored as whole records.
  const int rp_seq = lane >> 4, rp_row = (lane >> 1) & 7, rp_half = lane & 1;
  uint32_t orec[2];
  int lrec[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int sp = 4 * j + rp_seq;
    orec[j] = static_cast<uint32_t>(sp) * nbp * 256u + static_cast<uint32_t>(lane & 15) * 16u;
    lrec[j] = sp * 64 + ((rp_row + sp) & 7) * 8 + 4 * rp_half;
  }
  auto stage_ckpt = [&](uint32_t c) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      tile[FwdSlot::K + s * 64 + (((g ^ m) + s) & 7) * 8 + g] = b.Mv[m];
      tile[FwdSlot::D + s * 64 + ((g + s) & 7) * 8 + (g ^ m)] = b.P[m];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const v4f pm = *reinterpret_cast<const v4f*>(&tile[FwdSlot::K + lrec[j]]);
      const v4f pc = *reinterpret_cast<const v4f*>(&tile[FwdSlot::D + lrec[j]]);
      st128<0>(rbm, pm, orec[j], c * 256u);
      st128<0>(rbc, pc, orec[j], c * 256u);
    }
  };
  stage_ckpt(0);

  auto load = [&](FwdStage& x, uint32_t t0) __attribute__((always_inline)) {
    const bool full = static_cast<int64_t>(t0) + kFwdTile <= T;
    const bool in8 = full || static_cast<int64_t>(t0) + tok8 < T, in1 = full || static_cast<int64_t>(t0) + tok1 < T;
    const uint32_t s8 = t0 * 32u, s1 = t0 * 4u;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const uint32_t off = in8 ? o8[I] : kOob;
      x.k[I] = r4::ld128<kNt>(rk, off, s8);
      if constexpr (!FIXED) x.d[I] = r4::ld128<kNt>(rd, off, s8);
      x.q[I] = r4::ld128<kNt>(rq, off, s8);
      x.v[I] = r4::ld128<kNt>(rv, off, s8);
    }
    if constexpr (!FIXED) {
      const uint32_t off = (in1 && o1 != kOob) ? o1 : kOob;
      x.p = r4::ld128<false>(rp, off, s1);
      x.r = r4::ld128<false>(rr, off, s1);
    }
  };
  auto put = [&](const FwdStage& x) __attribute__((always_inline)) {
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      *reinterpret_cast<v4f*>(&tile[FwdSlot::K + l8[I]]) = x.k[I];
      if constexpr (!FIXED) *reinterpret_cast<v4f*>(&tile[FwdSlot::D + l8[I]]) = x.d[I];
      *reinterpret_cast<v4f*>(&tile[FwdSlot::Q + l8[I]]) = x.q[I];
      *reinterpret_cast<v4f*>(&tile[FwdSlot::V + l8[I]]) = x.v[I];
    }
    if constexpr (!FIXED) {
      if (lane < 32) {
        *reinterpret_cast<v4f*>(&tile[FwdSlot::P + 4 * lane]) = x.p;
        *reinterpret_cast<v4f*>(&tile[FwdSlot::R + 4 * lane]) = x.r;
      }
    }
  };
  auto read_tok = [&](int tt, Tok& x, float (&qx)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      x.kx[m] = tile[FwdSlot::K + 64 * tt + ix[m]];
      x.dx[m] = FIXED ? kFixedDecay : tile[FwdSlot::D + 64 * tt + ix[m]];
      qx[m] = tile[FwdSlot::Q + 64 * tt + ix[m]];
    }
    x.v = tile[FwdSlot::V + 64 * tt + ix[0]];
    x.p = FIXED ? kFixedProcess : tile[FwdSlot::P + 16 * s + tt];
    x.r = FIXED ? kFixedObservation : tile[FwdSlot::R + 16 * s + tt];
  };
  // One token: the step, then the readout y_g = sum_j M[j][g] q_j of the
  // mean after it, into the token's value slot.
  auto token = [&](int tt, const Tok& x, const float (&qx)[8]) __attribute__((always_inline)) {
    Hist h;
    step(b, x, a.floor, h);
    float y = b.Mv[0] * qx[0];
#pragma unroll
    for (int m = 1; m < 8; ++m) y = fmaf(b.Mv[m], qx[m], y);
    tile[FwdSlot::V + 64 * tt + ix[0]] = y;
  };

  const int64_t ntiles = (T + kFwdTile - 1) / kFwdTile;
  const bool fast = a.chunk % 8 == 0;
  int64_t next_ckpt = a.chunk;
  uint32_t ckpt = 1;
  FwdStage x;
  if (ntiles > 0) load(x, 0);
  v4f ys[4];
  for (int64_t ti = 0; ti < ntiles; ++ti) {
    const uint32_t t0 = static_cast<uint32_t>(ti) * kFwdTile;
    const int len = static_cast<int>((T - t0) < kFwdTile ? (T - t0) : kFwdTile);
    // The previous tile's readouts leave LDS before this tile lands there.
    if (ti > 0) {
#pragma unroll
      for (int I = 0; I < 4; ++I) ys[I] = *reinterpret_cast<const v4f*>(&tile[FwdSlot::V + l8[I]]);
    }
    vm_wait<0>();
    put(x);
    if (ti > 0) {
      const uint32_t s8 = (t0 - kFwdTile) * 32u;
#pragma unroll
      for (int I = 0; I < 4; ++I) st128<kNtSt>(ry, ys[I], o8[I], s8);
    }
    if (ti + 1 < ntiles) load(x, t0 + kFwdTile);
    lds_wait();
    if (fast) {
      // Records fall on 8-token boundaries (T is a multiple of 8); each is
      // staged after the token before it, over the spent first half.
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        if (hh * 8 >= len) break;
        Tok cur, nxt;
        float qc[8], qn[8];
        read_tok(8 * hh, cur, qc);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int tt = 8 * hh + u;
          if (u + 1 < 8) read_tok(tt + 1, nxt, qn);
          __builtin_amdgcn_sched_barrier(0);
          token(tt, cur, qc);
          __builtin_amdgcn_sched_barrier(0);
          cur = nxt;
#pragma unroll
          for (int m = 0; m < 8; ++m) qc[m] = qn[m];
        }
        const int64_t te = static_cast<int64_t>(t0) + 8 * (hh + 1);
        if (te == next_ckpt && te < T) {
          stage_ckpt(ckpt++);
          next_ckpt += a.chunk;
        }
      }
    } else {
      for (int tt = 0; tt < len; ++tt) {
        if (static_cast<int64_t>(t0) + tt == next_ckpt) {
          store_ckpt(ckpt++);
          next_ckpt += a.chunk;
        }
        Tok cur;
        float qc[8];
        read_tok(tt, cur, qc);
        token(tt, cur, qc);
      }
    }
  }
  if (ntiles > 0) {
    // The last tile's readouts (pieces of tokens past T are dropped).
    const uint32_t t0 = static_cast<uint32_t>(ntiles - 1) * kFwdTile;
    lds_wait();
    const bool in8 = static_cast<int64_t>(t0) + tok8 < T;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const v4f yv = *reinterpret_cast<const v4f*>(&tile[FwdSlot::V + l8[I]]);
      st128<kNtSt>(ry, yv, in8 ? o8[I] : kOob, t0 * 32u);
    }
  }
  const Rsrc rmT = make_rsrc(a.mT + n0 * 64, valid * 256u);
  const Rsrc rcT = make_rsrc(a.cT + n0 * 64, valid * 256u);
  store_bel(rmT, rcT, static_cast<uint32_t>(s) * 256u, 0);
  stage_ckpt(static_cast<uint32_t>(a.nb));
}

}  // namespace d8

// D = 8, M = 8 forward: T a positive multiple of 8, any checkpoint chunk,
// 16-byte aligned streams (the records are stored entry by entry).
bool d8_forward_ok(const FwdArgs& a) {
  return a.vec_kqd && a.vec_v && a.vec_pr && a.in_fmt == kInF32 && a.t > 0 && a.t % 8 == 0 &&
         a.t * 256 < (int64_t(1) << 31) && (a.nb + 1) * 2048 < (int64_t(1) << 31);
}

hipError_t launch_forward_d8(bool fixed, const FwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + d8::SPW - 1) / d8::SPW;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  if (fixed) hipLaunchKernelGGL((d8::forward_kernel<true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((d8::forward_kernel<false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

// D = 8, M = 8 with T a positive multiple of 8, the preferred checkpoint
// chunk (8), 16-byte aligned streams and 16-byte aligned checkpoint tensors.
bool d8_backward_ok(const BwdArgs& a) {
  const bool rec16 = (reinterpret_cast<uintptr_t>(a.bm) & 15u) == 0 && (reinterpret_cast<uintptr_t>(a.bc) & 15u) == 0;
  return a.vec_kqd && a.vec_v && a.vec_pr && rec16 && a.t > 0 && a.t % d8::kChunk == 0 && a.chunk == d8::kChunk &&
         a.t * 256 < (int64_t(1) << 31) && (a.nb + 1) * 2048 < (int64_t(1) << 31);
}

hipError_t launch_backward_d8(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + d8::SPW - 1) / d8::SPW;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  if (fixed) hipLaunchKernelGGL((d8::backward_kernel<true, false>), grid, block, 0, stream, a);
  else if (dyn) hipLaunchKernelGGL((d8::backward_kernel<false, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((d8::backward_kernel<false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace bssm
