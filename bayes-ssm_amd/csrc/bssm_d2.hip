// gfx950 forward and checkpoint-replay backward for D = 2, M = 8
// (bayes_ssm/persistent_bayes_chunked_d2m8.cu is the reference extension for
// this shape; the per-token equations are those of bssm_step.h with two key
// dimensions).  The forward streams its inputs as the generic kernels do
// (register-staged 16-token tiles, one tile ahead), one value column per
// lane: a version fed by 8-token LDS-DMA blocks measured slower, since this
// forward does little arithmetic per byte and needs more bytes in flight
// than such blocks leave.
//
// In the backward a wave holds 16 sequences; lane l = 4 s + g owns value
// columns 2g, 2g + 1 of sequence s.  Every lane carries the whole 2 x 2 covariance of its
// sequence (the four lanes apply the same operations to the same inputs, so
// they hold identical values; the two off-diagonal entries are carried
// separately, as the row owners of the generic kernels carry them), so the
// replay needs no cross-lane traffic and the reverse's sums over value
// columns are 4-lane DPP all-reduces.
//
// The backward's inputs arrive one block ahead, in blocks of 8 tokens (one
// checkpoint chunk): p, r and the checkpoint records by LDS-DMA; v and gy
// through registers, each load instruction requesting whole 256-byte row
// segments of four sequences (a DMA instruction could only fill the
// token-major layout from 64-byte pieces of 16 rows); k, d and q through
// registers per pair of blocks (16 tokens: whole 128-byte rows per sequence,
// each requested by one instruction; 8-token pieces are half lines, and
// their lines were fetched once per half).
// LDS layouts (floats):
//   k, d, q (two per token): piece-major [8 pieces][16 seq][2 tokens x 2]
//     per pair, in two pair buffers;
//   p, r: piece-major [2 pieces][16 seq][4 tokens] (the DMA instruction's
//     upper 32 lanes are idle and fill the padding after it with zeros);
//   v, gy: token-major [8][16 seq][8 col] with the sequences of token t in
//     XOR order (sequence s at position s ^ t), so lane l = 4 s + g reads
//     floats 128 t + 8 (s ^ t) + 2 g, + 1 of token t;
//   checkpoint records: mean [16 seq][2][8], covariance [16 seq][2][2]
//     (+ padding).
// Gradients overwrite their inputs in place and leave as 16-byte pieces
// through the same maps (dL/dv through the row-segment map of v).

#include "bssm_rot4.h"
#include "bssm_step.h"

namespace bssm {
namespace d2 {

using r4::dma16;
using r4::kOob;
using r4::make_rsrc;
using r4::Rsrc;
using r4::st128;
using r4::st64;
using r4::vm_wait;

typedef float v2f __attribute__((ext_vector_type(2)));

constexpr int SPW = 16;     // sequences per wave
constexpr int BT = 8;       // block, tokens
constexpr int kChunk = 8;   // backward checkpoint chunk, tokens
constexpr bool kNt = r4::kNtLoad;
constexpr int kNtSt = r4::kNtStore;

// Float offsets inside one block slot.
struct Slot {
  static constexpr int P = 0, R = 256, V = 512, GY = 1536, CKM = 2560, CKC = 2816;
  static constexpr int BWD = 3072;
};
// k, d, q of a pair of blocks (16 tokens: whole 128-byte rows per sequence),
// piece-major [8 pieces][16 seq][2 tokens x 2] per stream; block 2m + h of
// pair m reads pieces 4h .. 4h + 3.
struct KQ {
  static constexpr int K = 0, D = 512, Q = 1024, SIZE = 1536;
};

__device__ __forceinline__ v4f lds4(const float* p) { return *reinterpret_cast<const v4f*>(p); }
__device__ __forceinline__ v2f lds2(const float* p) { return *reinterpret_cast<const v2f*>(p); }
__device__ __forceinline__ void lds4_store(float* p, v4f x) { *reinterpret_cast<v4f*>(p) = x; }
__device__ __forceinline__ void lds2_store(float* p, v2f x) { *reinterpret_cast<v2f*>(p) = x; }

// Per-lane DMA / store offsets (bytes, relative to the wave's stream base)
// of a block starting at token t0.
struct Map {
  uint32_t s_base, s_piece;  // p/r: sequence j & 15, piece j >> 4 (4 tokens), lanes < 32
  __device__ __forceinline__ Map(int lane, uint32_t row1)
      : s_base(static_cast<uint32_t>(lane & 15) * row1), s_piece(static_cast<uint32_t>(lane >> 4)) {}
  __device__ __forceinline__ uint32_t s(uint32_t t0, uint32_t T) const {
    const uint32_t t = t0 + 4u * s_piece;
    return (s_piece < 2u && t < T) ? s_base + 4u * t : kOob;
  }
};

// Inputs of one token as lane (s, g) sees them.
struct Tok {
  float k[2], d[2], q[2], p, r;
  float v[2];
};

// Inputs of a 4-token piece: two k/d/q pieces, one p/r piece, four v pairs.
struct Piece {
  v4f k[2], d[2], q[2], p, r;
  v2f v[4];
  __device__ __forceinline__ Tok tok(int j) const {
    Tok t;
    const int h = j >> 1, o = 2 * (j & 1);
    t.k[0] = k[h][o];
    t.k[1] = k[h][o + 1];
    t.d[0] = d[h][o];
    t.d[1] = d[h][o + 1];
    t.q[0] = q[h][o];
    t.q[1] = q[h][o + 1];
    t.p = p[j];
    t.r = r[j];
    t.v[0] = v[j][0];
    t.v[1] = v[j][1];
    return t;
  }
};

// Piece pc (tokens 4 pc .. 4 pc + 3 of the block) of slot sl, with the
// block's k, d, q at kq (its half of the pair area).
template <bool FIXED>
__device__ __forceinline__ void read_piece(const float* sl, const float* kq, int pc, int seq, const int (&vsw)[8],
                                           bool need_v, bool need_q, Piece& x) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int o = 64 * (2 * pc + h) + 4 * seq;
    x.k[h] = lds4(kq + KQ::K + o);
    if constexpr (FIXED) x.d[h] = v4f{kFixedDecay, kFixedDecay, kFixedDecay, kFixedDecay};
    else x.d[h] = lds4(kq + KQ::D + o);
    if (need_q) x.q[h] = lds4(kq + KQ::Q + o);
  }
  if constexpr (FIXED) {
    x.p = v4f{kFixedProcess, kFixedProcess, kFixedProcess, kFixedProcess};
    x.r = v4f{kFixedObservation, kFixedObservation, kFixedObservation, kFixedObservation};
  } else {
    x.p = lds4(sl + Slot::P + 64 * pc + 4 * seq);
    x.r = lds4(sl + Slot::R + 64 * pc + 4 * seq);
  }
  if (need_v) {
#pragma unroll
    for (int j = 0; j < 4; ++j) x.v[j] = lds2(sl + Slot::V + 128 * (4 * pc + j) + vsw[4 * pc + j]);
  }
}

// Belief of one lane: the covariance (row-major, both off-diagonal entries)
// and the lane's two columns of both mean rows.
struct Bel {
  float P[4];
  float M[2][2];  // [row][own column]
};

// What the reverse of one token needs from its replay.
struct Hist {
  float P[4], M[2][2];  // belief before the token
  float u[2], s, e[2];  // u = P' k, s = r + k.u, own innovations
};

// One replayed token (the D = 2 case of forward_step in bssm_step.h: row i
// of the covariance update uses row i's entries only).
__device__ __forceinline__ void step(Bel& b, const Tok& x, float floor, Hist& h) {
  float dp[4], Pb[4], u[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float acc = x.p * x.k[i];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      dp[2 * i + j] = (x.d[i] * x.d[j]) * b.P[2 * i + j];
      Pb[2 * i + j] = fmaf(x.p, i == j ? 1.f : 0.f, dp[2 * i + j]);
      acc = fmaf(dp[2 * i + j], x.k[j], acc);
    }
    u[i] = acc;
  }
  const float s = fmaf(x.k[1], u[1], fmaf(x.k[0], u[0], x.r));
  const float beta = fast_rcp(fmaxf(s, floor));
  const float wk0 = x.d[0] * x.k[0], wk1 = x.d[1] * x.k[1];
  const float bu0 = beta * u[0], bu1 = beta * u[1];
#pragma unroll
  for (int i = 0; i < 4; ++i) h.P[i] = b.P[i];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    h.M[0][c] = b.M[0][c];
    h.M[1][c] = b.M[1][c];
    const float e = fmaf(-b.M[1][c], wk1, fmaf(-b.M[0][c], wk0, x.v[c]));
    h.e[c] = e;
    b.M[0][c] = fmaf(bu0, e, x.d[0] * b.M[0][c]);
    b.M[1][c] = fmaf(bu1, e, x.d[1] * b.M[1][c]);
  }
  h.u[0] = u[0];
  h.u[1] = u[1];
  h.s = s;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) b.P[2 * i + j] = fmaf(-beta, u[i] * u[j], Pb[2 * i + j]);
}

// Forward: the generic kernels' register-staged 16-token tiles (the next
// tile is loaded into registers while this one is computed, then written
// into padded LDS rows), with one value column per lane: 8 sequences per
// wave, so config 3's 16384 sequences give two waves per SIMD (with two
// columns per lane, one: 170 against 166 us).  The covariance chain is that
// of step() (every lane of a sequence carries it), and each column's mean
// update is that of step()'s column loop, so the backward's replay rebuilds
// the forward's beliefs bit for bit.  Each token's LDS reads are issued one
// token ahead.
constexpr int kFwdTile = 16;

struct FwdTok {
  v2f k, d, q, v;
  float p, r;
};

constexpr int SPW8 = 8;

struct Bel1 {
  float P[4];
  float M[2];  // rows 0, 1 of the lane's column
};

__device__ __forceinline__ void step1(Bel1& b, const FwdTok& x, float floor) {
  float dp[4], Pb[4], u[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float acc = x.p * x.k[i];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      dp[2 * i + j] = (x.d[i] * x.d[j]) * b.P[2 * i + j];
      Pb[2 * i + j] = fmaf(x.p, i == j ? 1.f : 0.f, dp[2 * i + j]);
      acc = fmaf(dp[2 * i + j], x.k[j], acc);
    }
    u[i] = acc;
  }
  const float s = fmaf(x.k[1], u[1], fmaf(x.k[0], u[0], x.r));
  const float beta = fast_rcp(fmaxf(s, floor));
  const float wk0 = x.d[0] * x.k[0], wk1 = x.d[1] * x.k[1];
  const float bu0 = beta * u[0], bu1 = beta * u[1];
  const float e = fmaf(-b.M[1], wk1, fmaf(-b.M[0], wk0, x.v[0]));
  b.M[0] = fmaf(bu0, e, x.d[0] * b.M[0]);
  b.M[1] = fmaf(bu1, e, x.d[1] * b.M[1]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) b.P[2 * i + j] = fmaf(-beta, u[i] * u[j], Pb[2 * i + j]);
}

template <bool FIXED>
__global__ __launch_bounds__(kWave) void forward8_kernel(FwdArgs a) {
  constexpr int TT = kFwdTile;
  constexpr int SD = Tile<2, TT>::STRIDE, SM = Tile<8, TT>::STRIDE, S1 = Tile<1, TT>::STRIDE;
  __shared__ float tk[SPW8 * SD];
  __shared__ float tq[SPW8 * SD];
  __shared__ float tv[SPW8 * SM];  // values in, readouts out (in place)
  __shared__ float td[FIXED ? 1 : SPW8 * SD];
  __shared__ float tp[FIXED ? 1 : SPW8 * S1];
  __shared__ float tr[FIXED ? 1 : SPW8 * S1];
  const int lane = threadIdx.x;
  const int seq = lane >> 3, g = lane & 7;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW8;
  const int64_t T = a.t;
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW8 ? (a.n - n0) : SPW8);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 16, valid * nbp * 64u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 4, valid * nbp * 16u);
  // Belief record offsets of this lane: its column of both mean rows (the 8
  // lanes of a sequence write each 32-byte row together), and the
  // covariance record (written by lane 0 of the sequence).
  const uint32_t bm_off = static_cast<uint32_t>(seq) * nbp * 64u + 4u * g;
  const uint32_t bc_off = g == 0 ? static_cast<uint32_t>(seq) * nbp * 16u : kOob;

  Bel1 b;
  {
    const Rsrc rm0 = make_rsrc(a.m0 + n0 * 16, valid * 64u);
    const Rsrc rc0 = make_rsrc(a.c0 + n0 * 4, valid * 16u);
    const uint32_t mo = static_cast<uint32_t>(seq) * 64u + 4u * g;
    b.M[0] = r4::ld32(rm0, mo, 0);
    b.M[1] = r4::ld32(rm0, mo + 32u, 0);
    const v4f c = r4::ld128<false>(rc0, static_cast<uint32_t>(seq) * 16u);
#pragma unroll
    for (int i = 0; i < 4; ++i) b.P[i] = c[i];
  }
  auto store_bel = [&](Rsrc rm, Rsrc rc, uint32_t moff, uint32_t coff, uint32_t soff_m, uint32_t soff_c)
      __attribute__((always_inline)) {
    r4::st32(rm, b.M[0], moff, soff_m);
    r4::st32(rm, b.M[1], moff + 32u, soff_m);
    st128(rc, v4f{b.P[0], b.P[1], b.P[2], b.P[3]}, coff, soff_c);
  };
  store_bel(rbm, rbc, bm_off, bc_off, 0, 0);

  TileRegs<2, TT, SPW8> rk, rq, rd;
  TileRegs<8, TT, SPW8> rv;
  TileRegs<1, TT, SPW8> rp, rr;
  auto issue = [&](int64_t t0) __attribute__((always_inline)) {
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
  if (T > 0) issue(0);
  const float* sk = tk + seq * SD;
  const float* sq = tq + seq * SD;
  float* sv = tv + seq * SM;
  const float* sd = FIXED ? tk : td + seq * SD;
  const float* sp = FIXED ? tk : tp + seq * S1;
  const float* sr = FIXED ? tk : tr + seq * S1;
  auto read = [&](int tt) __attribute__((always_inline)) {
    FwdTok x;
    x.k = lds2(sk + 2 * tt);
    x.q = lds2(sq + 2 * tt);
    x.v[0] = sv[8 * tt + g];
    if constexpr (FIXED) {
      x.d = v2f{kFixedDecay, kFixedDecay};
      x.p = kFixedProcess;
      x.r = kFixedObservation;
    } else {
      x.d = lds2(sd + 2 * tt);
      x.p = sp[tt];
      x.r = sr[tt];
    }
    return x;
  };
  const uint32_t chunk = static_cast<uint32_t>(a.chunk);
  uint32_t next_ckpt = chunk, ckpt = 1;
  for (int64_t t0 = 0; t0 < T; t0 += TT) {
    const int len = tile_len(T, t0, TT);
    rk.commit(tk, lane);
    rq.commit(tq, lane);
    rv.commit(tv, lane);
    if constexpr (!FIXED) {
      rd.commit(td, lane);
      rp.commit(tp, lane);
      rr.commit(tr, lane);
    }
    __syncthreads();
    if (t0 + TT < T) issue(t0 + TT);
    FwdTok cur = read(0);
    for (int tt = 0; tt < len; ++tt) {
      const FwdTok nxt = read(tt + 1 < len ? tt + 1 : tt);
      if (static_cast<uint32_t>(t0) + tt == next_ckpt) {
        store_bel(rbm, rbc, bm_off, bc_off, ckpt * 64u, ckpt * 16u);
        ++ckpt;
        next_ckpt += chunk;
      }
      step1(b, cur, a.floor);
      sv[8 * tt + g] = fmaf(b.M[1], cur.q[1], fmaf(b.M[0], cur.q[0], 0.f));
      cur = nxt;
    }
    __syncthreads();
    stage_out<8, TT, SPW8>(tv, a.y, n0, a.n, T, t0, len, true, lane);
    __syncthreads();
  }
  store_bel(make_rsrc(a.mT + n0 * 16, valid * 64u), make_rsrc(a.cT + n0 * 4, valid * 16u),
            static_cast<uint32_t>(seq) * 64u + 4u * g, g == 0 ? static_cast<uint32_t>(seq) * 16u : kOob, 0, 0);
  if (T > 0) {
    const uint32_t nb = static_cast<uint32_t>(a.nb);
    store_bel(rbm, rbc, bm_off, bc_off, nb * 64u, nb * 16u);
  }
}

// Sum over the 4 lanes (column pairs) of the caller's sequence.
__device__ __forceinline__ float colsum(float x) { return group_sum<4>(x); }

// Token outputs of the reverse (per-sequence values identical on the 4 lanes).
struct RevOut2 {
  float gk[2], gq[2], gd[2], gp, gr;
  float gv[2];
};

// Reverse of one token (the D = 2, two-columns-per-lane case of
// reverse_step in bssm_step.h).  gM: own columns of dL/dM; Gs: sym(dL/dP)
// (G00, G01, G11).  At the first token the full (asymmetric) adjoint of the
// initial covariance is left in gc0.
template <bool DYN>
__device__ __forceinline__ void reverse(const Hist& h, const Tok& x, float floor, float (&gM)[2][2],
                                        float (&Gs)[3], bool first, float (&gc0)[4], RevOut2& o) {
  const float beta = fast_rcp(fmaxf(h.s, floor));
  float mp[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c) mp[i][c] = x.d[i] * h.M[i][c];
  float Pb[4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) Pb[2 * i + j] = fmaf(x.p, i == j ? 1.f : 0.f, (x.d[i] * x.d[j]) * h.P[2 * i + j]);

  float gqp[2] = {0.f, 0.f}, ap[2] = {0.f, 0.f}, gkp[2] = {0.f, 0.f}, gdp[2] = {0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float bu = beta * h.u[i];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      gqp[i] = fmaf(fmaf(bu, h.e[c], mp[i][c]), x.v[c], gqp[i]);  // x.v holds gy here
      gM[i][c] = fmaf(x.q[i], x.v[c], gM[i][c]);
    }
  }
  float ge[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    ge[c] = beta * fmaf(gM[1][c], h.u[1], fmaf(gM[0][c], h.u[0], 0.f));
    o.gv[c] = ge[c];
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      ap[i] = fmaf(gM[i][c], h.e[c], ap[i]);
      gkp[i] = fmaf(-mp[i][c], ge[c], gkp[i]);
      const float gmb = fmaf(-x.k[i], ge[c], gM[i][c]);
      if constexpr (DYN) gdp[i] = fmaf(gmb, h.M[i][c], gdp[i]);
      gM[i][c] = gmb * x.d[i];
    }
  float av[2], gkc[2], gdc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    av[i] = colsum(ap[i]);
    gkc[i] = colsum(gkp[i]);
    o.gq[i] = colsum(gqp[i]);
    gdc[i] = DYN ? colsum(gdp[i]) : 0.f;
  }
  const float G[2][2] = {{Gs[0], Gs[1]}, {Gs[1], Gs[2]}};
  float w[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) w[i] = fmaf(G[i][1], h.u[1], fmaf(G[i][0], h.u[0], 0.f));
  const float z = fmaf(h.u[0], av[0] - w[0], 0.f) + fmaf(h.u[1], av[1] - w[1], 0.f);
  const float gs = (h.s > floor) ? -z * beta * beta : 0.f;
  float gu[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) gu[i] = fmaf(beta, av[i] - 2.f * w[i], gs * x.k[i]);
  float hs[2][2], gd[2] = {0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float gk = fmaf(gs, h.u[i], gkc[i]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      gk = fmaf(Pb[2 * i + j], gu[j], gk);
      hs[i][j] = fmaf(0.5f, gu[i] * x.k[j] + gu[j] * x.k[i], G[i][j]);
      if constexpr (DYN) gd[i] = fmaf(hs[i][j] * x.d[j], h.P[2 * i + j], gd[i]);
      if (first) gc0[2 * i + j] = fmaf(gu[i], x.k[j], G[i][j]) * (x.d[i] * x.d[j]);
    }
    o.gk[i] = gk;
    o.gd[i] = DYN ? fmaf(2.f, gd[i], gdc[i]) : 0.f;
  }
  Gs[0] = hs[0][0] * (x.d[0] * x.d[0]);
  Gs[1] = hs[0][1] * (x.d[0] * x.d[1]);
  Gs[2] = hs[1][1] * (x.d[1] * x.d[1]);
  o.gp = DYN ? hs[0][0] + hs[1][1] : 0.f;
  o.gr = DYN ? gs : 0.f;
}

template <bool FIXED, bool DYN>
__global__ __launch_bounds__(kWave) void backward_kernel(BwdArgs a) {
  __shared__ float tile[2 * Slot::BWD];
  __shared__ float kdq[2 * KQ::SIZE];
  const int lane = threadIdx.x;
  const int seq = lane >> 2, g = lane & 3;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const uint32_t T = static_cast<uint32_t>(a.t);
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  const uint32_t row1 = T * 4u, row2 = T * 8u, row8 = T * 32u;
  const Rsrc rk = make_rsrc(a.k + n0 * T * 2, valid * row2);
  const Rsrc rq = make_rsrc(a.q + n0 * T * 2, valid * row2);
  const Rsrc rv = make_rsrc(a.v + n0 * T * 8, valid * row8);
  const Rsrc rgy = make_rsrc(a.gy + n0 * T * 8, valid * row8);
  const Rsrc rd = make_rsrc(FIXED ? a.k : a.d + n0 * T * 2, FIXED ? 0u : valid * row2);
  const Rsrc rp = make_rsrc(FIXED ? a.k : a.p + n0 * T, FIXED ? 0u : valid * row1);
  const Rsrc rr = make_rsrc(FIXED ? a.k : a.r + n0 * T, FIXED ? 0u : valid * row1);
  const Rsrc rgk = make_rsrc(a.gk + n0 * T * 2, valid * row2);
  const Rsrc rgq = make_rsrc(a.gq + n0 * T * 2, valid * row2);
  const Rsrc rgv = make_rsrc(a.gv + n0 * T * 8, valid * row8);
  const Rsrc rgd = make_rsrc(a.gd ? a.gd + n0 * T * 2 : a.gk, a.gd ? valid * row2 : 0u);
  const Rsrc rgp = make_rsrc(a.gp ? a.gp + n0 * T : a.gk, a.gp ? valid * row1 : 0u);
  const Rsrc rgr = make_rsrc(a.gr ? a.gr + n0 * T : a.gk, a.gr ? valid * row1 : 0u);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 16, valid * nbp * 64u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 4, valid * nbp * 16u);
  const Map mp(lane, row1);
  // Checkpoint record DMA: mean records by (sequence j >> 2, piece j & 3),
  // covariance records by lanes j < 16.
  const uint32_t ckm_off = static_cast<uint32_t>(lane >> 2) * nbp * 64u + 16u * (lane & 3);
  const uint32_t ckc_off = lane < 16 ? static_cast<uint32_t>(lane) * nbp * 16u : kOob;

  // Carried adjoints: gM = dL/dM (own columns), Gs = sym(dL/dP).
  float gM[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  float Gs[3] = {0.f, 0.f, 0.f};
  if (a.gmf) {
    const Rsrc r = make_rsrc(a.gmf + n0 * 16, valid * 64u);
    const uint32_t mo = static_cast<uint32_t>(seq) * 64u + 8u * g;
    const v2f m0 = r4::ld64(r, mo, 0), m1 = r4::ld64(r, mo + 32u, 0);
    gM[0][0] = m0[0];
    gM[0][1] = m0[1];
    gM[1][0] = m1[0];
    gM[1][1] = m1[1];
  }
  v4f gcf = v4f{0.f, 0.f, 0.f, 0.f};
  if (a.gcf) {
    gcf = r4::ld128<false>(make_rsrc(a.gcf + n0 * 4, valid * 16u), static_cast<uint32_t>(seq) * 16u);
    Gs[0] = 0.5f * (gcf[0] + gcf[0]);
    Gs[1] = 0.5f * (gcf[1] + gcf[2]);
    Gs[2] = 0.5f * (gcf[3] + gcf[3]);
  }
  float gc0[4] = {0.f, 0.f, 0.f, 0.f};

  // v, gy and dL/dv move as whole 256-byte row segments: load instruction
  // I < 4, lane l -> sequence 4 I + (l >> 4), piece l & 15 (token
  // (l & 15) >> 1, half l & 1) of the block, staged in registers one block
  // ahead and written into the XOR-ordered token-major layout (4-way bank
  // use per write, the minimum for 16-byte writes).
  const int vt = (lane & 15) >> 1;
  uint32_t vo[4];
  int vl[4];
#pragma unroll
  for (int I = 0; I < 4; ++I) {
    const int sq = 4 * I + (lane >> 4);
    vo[I] = static_cast<uint32_t>(sq) * row8 + static_cast<uint32_t>(lane & 15) * 16u;
    vl[I] = 128 * vt + 8 * (sq ^ vt) + 4 * (lane & 1);
  }
  // Per-token offsets of the lane's own pair (token t of a block).
  int vsw[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) vsw[t] = 8 * (seq ^ t) + 2 * g;
  v4f sv[4], sgy[4];
  auto load_v = [&](uint32_t blk) __attribute__((always_inline)) {
    const uint32_t t0 = blk * BT;
    const bool in = t0 + static_cast<uint32_t>(vt) < T;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const uint32_t off = in ? vo[I] : kOob;
      sv[I] = r4::ld128<kNt>(rv, off, t0 * 32u);
      sgy[I] = r4::ld128<kNt>(rgy, off, t0 * 32u);
    }
  };
  auto put_v = [&](float* sl) __attribute__((always_inline)) {
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      lds4_store(sl + Slot::V + vl[I], sv[I]);
      lds4_store(sl + Slot::GY + vl[I], sgy[I]);
    }
  };

  const uint32_t nblk = (T + BT - 1) / BT;
  // k, d, q of pair m, staged in registers a pair ahead: instruction i,
  // lane j covers piece j & 7 (2 tokens) of sequence 8 i + (j >> 3), so each
  // sequence's 128-byte row is requested by 8 lanes of one instruction.
  const int kq_piece = lane & 7;
  uint32_t kq_row[2];
  int kq_lds[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int sq = 8 * i + (lane >> 3);
    kq_row[i] = static_cast<uint32_t>(sq) * row2 + 16u * static_cast<uint32_t>(kq_piece);
    kq_lds[i] = 64 * kq_piece + 4 * sq;
  }
  v4f skk[2], sqq[2], sdd[2];
  auto load_kq = [&](uint32_t m) __attribute__((always_inline)) {
    const bool in = 16u * m + 2u * static_cast<uint32_t>(kq_piece) < T;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t off = in ? kq_row[i] : kOob;
      skk[i] = r4::ld128<kNt>(rk, off, 128u * m);
      sqq[i] = r4::ld128<kNt>(rq, off, 128u * m);
      if constexpr (!FIXED) sdd[i] = r4::ld128<kNt>(rd, off, 128u * m);
    }
  };
  auto put_kq = [&](float* kb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      lds4_store(kb + KQ::K + kq_lds[i], skk[i]);
      lds4_store(kb + KQ::Q + kq_lds[i], sqq[i]);
      if constexpr (!FIXED) lds4_store(kb + KQ::D + kq_lds[i], sdd[i]);
    }
  };
  auto store_kq = [&](const float* kb, uint32_t m) __attribute__((always_inline)) {
    const v4f zero = v4f{0.f, 0.f, 0.f, 0.f};
    const bool in = 16u * m + 2u * static_cast<uint32_t>(kq_piece) < T;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t off = in ? kq_row[i] : kOob;
      st128<kNtSt>(rgk, lds4(kb + KQ::K + kq_lds[i]), off, 128u * m);
      st128<kNtSt>(rgq, lds4(kb + KQ::Q + kq_lds[i]), off, 128u * m);
      st128<kNtSt>(rgd, DYN ? lds4(kb + KQ::D + kq_lds[i]) : zero, off, 128u * m);
    }
  };
  auto issue = [&](float* sl, uint32_t blk) __attribute__((always_inline)) {
    const uint32_t t0 = blk * BT;
    if constexpr (!FIXED) {
      const uint32_t os = mp.s(t0, T);
      dma16(rp, sl + Slot::P, os);
      dma16(rr, sl + Slot::R, os);
    }
    dma16(rbm, sl + Slot::CKM, ckm_off + 64u * blk);
    dma16(rbc, sl + Slot::CKC, ckc_off == kOob ? kOob : ckc_off + 16u * blk);
  };

  auto store_grads = [&](const float* sl, uint32_t blk) __attribute__((always_inline)) {
    const uint32_t t0 = blk * BT;
    const int e = 4 * lane;
    const v4f zero = v4f{0.f, 0.f, 0.f, 0.f};
    const uint32_t os = mp.s(t0, T);
    st128(rgp, DYN ? lds4(sl + Slot::P + e) : zero, os, 0);
    st128(rgr, DYN ? lds4(sl + Slot::R + e) : zero, os, 0);
    const bool in = t0 + static_cast<uint32_t>(vt) < T;
#pragma unroll
    for (int I = 0; I < 4; ++I) st128<kNtSt>(rgv, lds4(sl + Slot::V + vl[I]), in ? vo[I] : kOob, t0 * 32u);
  };

  // Replay the block's chunk from its checkpoint record, then reverse it;
  // the gradients overwrite the block's inputs.
  auto run_chunk = [&](float* sl, float* kq, int npc, bool first_chunk) __attribute__((always_inline)) {
    Bel b;
    {
      const v2f m0 = lds2(sl + Slot::CKM + 16 * seq + 2 * g), m1 = lds2(sl + Slot::CKM + 16 * seq + 8 + 2 * g);
      b.M[0][0] = m0[0];
      b.M[0][1] = m0[1];
      b.M[1][0] = m1[0];
      b.M[1][1] = m1[1];
      const v4f c = lds4(sl + Slot::CKC + 4 * seq);
#pragma unroll
      for (int i = 0; i < 4; ++i) b.P[i] = c[i];
    }
    Piece x[2];
    v2f gy[2][4];
#pragma unroll
    for (int pc = 0; pc < 2; ++pc) {
      read_piece<FIXED>(sl, kq, pc, seq, vsw, true, true, x[pc]);
#pragma unroll
      for (int j = 0; j < 4; ++j) gy[pc][j] = lds2(sl + Slot::GY + 128 * (4 * pc + j) + vsw[4 * pc + j]);
    }
    Hist h[kChunk];
#pragma unroll
    for (int pc = 0; pc < 2; ++pc)
      if (pc < npc)
#pragma unroll
        for (int j = 0; j < 4; ++j) step(b, x[pc].tok(j), a.floor, h[4 * pc + j]);
#pragma unroll
    for (int pc = 1; pc >= 0; --pc) {
      if (pc < npc) {
        v4f gk[2], gq[2], gd[2], gp, gr;
#pragma unroll
        for (int j = 3; j >= 0; --j) {
          Tok t = x[pc].tok(j);
          t.v[0] = gy[pc][j][0];
          t.v[1] = gy[pc][j][1];
          RevOut2 o;
          reverse<DYN>(h[4 * pc + j], t, a.floor, gM, Gs, first_chunk && pc == 0 && j == 0, gc0, o);
          const int hh = j >> 1, oo = 2 * (j & 1);
          gk[hh][oo] = o.gk[0];
          gk[hh][oo + 1] = o.gk[1];
          gq[hh][oo] = o.gq[0];
          gq[hh][oo + 1] = o.gq[1];
          gd[hh][oo] = o.gd[0];
          gd[hh][oo + 1] = o.gd[1];
          gp[j] = o.gp;
          gr[j] = o.gr;
          lds2_store(sl + Slot::V + 128 * (4 * pc + j) + vsw[4 * pc + j], v2f{o.gv[0], o.gv[1]});
        }
        if (g == 0) {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int o = 64 * (2 * pc + hh) + 4 * seq;
            lds4_store(kq + KQ::K + o, gk[hh]);
            lds4_store(kq + KQ::Q + o, gq[hh]);
            if constexpr (DYN) lds4_store(kq + KQ::D + o, gd[hh]);
          }
          if constexpr (DYN) {
            lds4_store(sl + Slot::P + 64 * pc + 4 * seq, gp);
            lds4_store(sl + Slot::R + 64 * pc + 4 * seq, gr);
          }
        }
      }
    }
  };

  // Block b is processed in slot b % 2.  At its start every outstanding
  // memory operation was issued at least a whole block earlier; then the
  // gradients of block b + 1 leave the other slot, which receives block
  // b - 1.  The k, d, q of pair m (blocks 2m, 2m + 1) live in pair buffer
  // m % 2: at the first block of pair m processed, pair m's k, d, q (staged
  // in registers during pair m + 1) land there and the loads of pair m - 1
  // are issued; the gradients of pair m + 1 leave the other buffer.
  const uint32_t npair = (nblk + 1) / 2;
  auto kbuf = [&](uint32_t m) __attribute__((always_inline)) { return kdq + (m & 1) * KQ::SIZE; };
  if (nblk > 0) {
    issue(tile + ((nblk - 1) & 1) * Slot::BWD, nblk - 1);
    load_kq(npair - 1);
    load_v(nblk - 1);
  }
  for (uint32_t i = 0; i < nblk; ++i) {
    const uint32_t blk = nblk - 1 - i, m = blk >> 1;
    float* cur = tile + (blk & 1) * Slot::BWD;
    float* other = tile + ((blk + 1) & 1) * Slot::BWD;
    vm_wait<0>();
    __syncthreads();
    put_v(cur);
    if (blk > 0) load_v(blk - 1);
    if (blk + 1 < nblk) store_grads(other, blk + 1);
    if (blk == nblk - 1 || (blk & 1) == 1) {  // first block of pair m
      put_kq(kbuf(m));
      if (m > 0) load_kq(m - 1);
      if (m + 1 < npair) store_kq(kbuf(m + 1), m + 1);
    }
    if (blk > 0) issue(other, blk - 1);
    run_chunk(cur, kbuf(m) + 256 * (blk & 1), (T - blk * BT) < BT ? 1 : 2, blk == 0);
  }
  if (nblk > 0) {
    __syncthreads();
    store_grads(tile, 0);
    store_kq(kbuf(0), 0);
  }
  if (a.gm0) {
    const Rsrc r = make_rsrc(a.gm0 + n0 * 16, valid * 64u);
    const uint32_t mo = static_cast<uint32_t>(seq) * 64u + 8u * g;
    st64(r, v2f{gM[0][0], gM[0][1]}, mo, 0);
    st64(r, v2f{gM[1][0], gM[1][1]}, mo + 32u, 0);
  }
  if (a.gc0)
    st128(make_rsrc(a.gc0 + n0 * 4, valid * 16u), T > 0 ? v4f{gc0[0], gc0[1], gc0[2], gc0[3]} : gcf,
          g == 0 ? static_cast<uint32_t>(seq) * 16u : kOob, 0);
}

}  // namespace d2

bool d2_forward_ok(const FwdArgs& a) {
  return a.vec_kqd && a.vec_v && a.vec_pr && a.t % 4 == 0 && a.chunk < (int64_t(1) << 30) &&
         (a.nb + 1) * 1024 < (int64_t(1) << 31);
}

bool d2_backward_ok(const BwdArgs& a) {
  return a.vec_kqd && a.vec_v && a.vec_pr && a.t > 0 && a.t % 4 == 0 && a.chunk == d2::kChunk &&
         a.t * 512 < (int64_t(1) << 31) && (a.nb + 1) * 1024 < (int64_t(1) << 31);
}

hipError_t launch_forward_d2(bool fixed, const FwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + d2::SPW8 - 1) / d2::SPW8;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  if (fixed) hipLaunchKernelGGL((d2::forward8_kernel<true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((d2::forward8_kernel<false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_backward_d2(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + d2::SPW - 1) / d2::SPW;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  if (fixed) hipLaunchKernelGGL((d2::backward_kernel<true, false>), grid, block, 0, stream, a);
  else if (dyn) hipLaunchKernelGGL((d2::backward_kernel<false, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((d2::backward_kernel<false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace bssm
