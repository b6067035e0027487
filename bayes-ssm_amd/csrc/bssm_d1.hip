// gfx950 kernels for D = 1, M = 8 (bayes_ssm/persistent_bayes_chunked_d1m8.cu
// is the reference extension for this shape; the per-token equations are
// those of bssm_step.h with one key dimension): the float32 forward and the
// checkpoint-replay backward with one lane per value column.
//
// A wave holds 8 sequences; lane l = 8 s + c owns value column c of sequence
// s.  With one key dimension the covariance is a scalar that all 8 lanes of
// a sequence carry with identical values (they apply the same operations to
// the same inputs), so the forward needs no cross-lane traffic at all and the
// backward's sums over value columns are 8-lane DPP all-reduces.  Each
// sequence is one serial chain of a few dependent operations per token, so a
// wave's time is its instruction stream: everything that is not arithmetic
// (staging, address work, checkpoint bookkeeping) is kept off the per-token
// path.
//
// Inputs arrive by LDS-DMA (16-byte pieces straight into LDS), one block
// ahead of the block being computed: 64 tokens in the forward, 32 (two
// 16-token checkpoint chunks) in the backward.  LDS layouts of a block of B
// tokens (floats):
//   per-token scalars k, d, q, p, r: piece-major [B/4][8 seq][4 tokens], so
//     the 8 sequences' 16-byte reads of one 4-token piece are contiguous;
//   value-width streams v, gy: token-major [B][8 seq][8 col], so lane l
//     reads word 64 t + l for token t.
// Readouts and gradients overwrite their inputs in place and leave as
// 16-byte pieces through the same maps.

#include "bssm_rot4.h"
#include "bssm_step.h"

namespace bssm {
namespace d1 {

using r4::dma16;
using r4::kOob;
using r4::ld32;
using r4::make_rsrc;
using r4::Rsrc;
using r4::st128;
using r4::st32;
using r4::vm_wait;

constexpr int SPW = 8;     // sequences per wave
constexpr int FB = 64;     // forward block, tokens
constexpr int BB = 32;     // backward block, tokens
constexpr int kChunk = 16; // backward checkpoint chunk, tokens
constexpr bool kNt = r4::kNtLoad;
constexpr int kNtSt = r4::kNtStore;

// Float offsets inside one block slot.
template <int B>
struct Slot {
  static constexpr int SC = 8 * B;  // one scalar stream
  static constexpr int K = 0, D = SC, Q = 2 * SC, P = 3 * SC, R = 4 * SC, V = 5 * SC, GY = V + 64 * B;
};
constexpr int kFwdSlot = Slot<FB>::V + 64 * FB;        // 6656 floats
// Forward ring of block slots: DMA up to kFwdSlots - 1 blocks ahead (a
// three-slot ring measured no faster at config 2).
constexpr int kFwdSlots = 2;
static_assert(kFwdSlots == 2 || kFwdSlots == 3, "forward ring size");
constexpr int kBwdSlot = Slot<BB>::GY + 64 * BB;       // 5376 floats

// Per-lane DMA / store offsets of one block (bytes, relative to the wave's
// stream base).  Scalar streams: instruction i, lane j covers piece
// 8 i + (j >> 3) of sequence j & 7.  Value-width streams: instruction i,
// lane j covers token 4 i + (j >> 4), sequence (j >> 1) & 7, half j & 1.
struct Map {
  uint32_t sc_base, sc_piece;  // sequence row offset, piece index within an instruction
  uint32_t v_base, v_tok;      // sequence row offset + half, token within an instruction
  __device__ __forceinline__ Map(int lane, uint32_t row1, uint32_t row8)
      : sc_base(static_cast<uint32_t>(lane & 7) * row1),
        sc_piece(static_cast<uint32_t>(lane >> 3)),
        v_base(static_cast<uint32_t>((lane >> 1) & 7) * row8 + static_cast<uint32_t>(lane & 1) * 16u),
        v_tok(static_cast<uint32_t>(lane >> 4)) {}
  // Scalar piece of instruction i for the block at token t0.
  __device__ __forceinline__ uint32_t sc(int i, uint32_t t0, uint32_t T) const {
    const uint32_t t = t0 + 4u * (8u * i + sc_piece);
    return t < T ? sc_base + 4u * t : kOob;
  }
  __device__ __forceinline__ uint32_t v(int i, uint32_t t0, uint32_t T) const {
    const uint32_t t = t0 + 4u * i + v_tok;
    return t < T ? v_base + 32u * t : kOob;
  }
};

__device__ __forceinline__ v4f lds4(const float* p) { return *reinterpret_cast<const v4f*>(p); }
__device__ __forceinline__ void lds4_store(float* p, v4f x) { *reinterpret_cast<v4f*>(p) = x; }

// Inputs of one 4-token piece as lane (s, c) sees them.
struct Piece {
  v4f k, d, p, r, q;
  float v[4];
};

template <int B, bool FIXED>
__device__ __forceinline__ void read_piece(const float* sl, int pc, int seq, int lane, bool need_v, bool need_q,
                                           Piece& x) {
  using S = Slot<B>;
  const int o = 32 * pc + 4 * seq;
  x.k = lds4(sl + S::K + o);
  if constexpr (FIXED) {
    x.d = v4f{kFixedDecay, kFixedDecay, kFixedDecay, kFixedDecay};
    x.p = v4f{kFixedProcess, kFixedProcess, kFixedProcess, kFixedProcess};
    x.r = v4f{kFixedObservation, kFixedObservation, kFixedObservation, kFixedObservation};
  } else {
    x.d = lds4(sl + S::D + o);
    x.p = lds4(sl + S::P + o);
    x.r = lds4(sl + S::R + o);
  }
  if (need_q) x.q = lds4(sl + S::Q + o);
  if (need_v) {
#pragma unroll
    for (int j = 0; j < 4; ++j) x.v[j] = sl[S::V + 64 * (4 * pc + j) + lane];
  }
}

// What the reverse of one token needs from its replay.
struct Hist {
  float P, M, u, s, e;  // covariance and own mean column before the token, u = P' k, s, innovation
};

// One forward token (the D = 1 case of forward_step in bssm_step.h; P is the
// scalar covariance, M the lane's mean column).
__device__ __forceinline__ void step(float& P, float& M, float k, float d, float p, float r, float v, float floor,
                                     Hist& h) {
  const float dp = (d * d) * P;
  const float Pb = fmaf(p, 1.f, dp);
  const float u = fmaf(dp, k, p * k);
  const float s = fmaf(k, u, r);
  const float beta = fast_rcp(fmaxf(s, floor));
  const float e = fmaf(-M, d * k, v);
  h.P = P;
  h.M = M;
  h.u = u;
  h.s = s;
  h.e = e;
  M = fmaf(beta * u, e, d * M);
  P = fmaf(-beta, u * u, Pb);
}

template <bool FIXED>
__global__ __launch_bounds__(kWave) void forward_kernel(FwdArgs a) {
  __shared__ float tile[kFwdSlots * kFwdSlot];
  using S = Slot<FB>;
  const int lane = threadIdx.x;
  const int seq = lane >> 3, col = lane & 7;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const uint32_t T = static_cast<uint32_t>(a.t);
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  const uint32_t row1 = T * 4u, row8 = T * 32u;
  const Rsrc rk = make_rsrc(a.k + n0 * T, valid * row1);
  const Rsrc rq = make_rsrc(a.q + n0 * T, valid * row1);
  const Rsrc rv = make_rsrc(a.v + n0 * T * 8, valid * row8);
  const Rsrc ry = make_rsrc(a.y + n0 * T * 8, valid * row8);
  const Rsrc rd = make_rsrc(FIXED ? a.y : a.d + n0 * T, FIXED ? 0u : valid * row1);
  const Rsrc rp = make_rsrc(FIXED ? a.y : a.p + n0 * T, FIXED ? 0u : valid * row1);
  const Rsrc rr = make_rsrc(FIXED ? a.y : a.r + n0 * T, FIXED ? 0u : valid * row1);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 8, valid * nbp * 32u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp, valid * nbp * 4u);
  const Map mp(lane, row1, row8);
  // Belief record offsets of this lane: mean column, and the covariance
  // (written by column 0 only).
  const uint32_t bm_off = static_cast<uint32_t>(seq) * nbp * 32u + 4u * col;
  const uint32_t bc_off = col == 0 ? static_cast<uint32_t>(seq) * nbp * 4u : kOob;

  float M = ld32(make_rsrc(a.m0 + n0 * 8, valid * 32u), 4u * lane, 0);
  float P = ld32(make_rsrc(a.c0 + n0, valid * 4u), 4u * seq, 0);
  st32(rbm, M, bm_off, 0);
  st32(rbc, P, bc_off, 0);

  auto issue = [&](float* sl, uint32_t t0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t off = mp.sc(i, t0, T);
      dma16<kNt>(rk, sl + S::K + 256 * i, off);
      dma16<kNt>(rq, sl + S::Q + 256 * i, off);
      if constexpr (!FIXED) {
        dma16<kNt>(rd, sl + S::D + 256 * i, off);
        dma16<kNt>(rp, sl + S::P + 256 * i, off);
        dma16<kNt>(rr, sl + S::R + 256 * i, off);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) dma16<kNt>(rv, sl + S::V + 256 * i, mp.v(i, t0, T));
  };
  constexpr int kLoads = FIXED ? 2 * 2 + 16 : 2 * 5 + 16;  // DMA instructions per block

  const uint32_t nblk = (T + FB - 1) / FB;
#pragma unroll
  for (int i = 0; i < kFwdSlots; ++i)
    if (static_cast<uint32_t>(i) < nblk) issue(tile + i * kFwdSlot, i * FB);
  const uint32_t chunk = static_cast<uint32_t>(a.chunk);
  uint32_t next_ckpt = chunk, ckpt = 1;
  for (uint32_t b = 0; b < nblk; ++b) {
    float* sl = tile + (b % kFwdSlots) * kFwdSlot;
    // Loads finish in issue order, so once at most the DMA of the blocks
    // after this one is outstanding this block's has landed.
    if (kFwdSlots > 2 && b + 2 < nblk) vm_wait<(kFwdSlots > 2 ? 2 : 1) * kLoads>();
    else if (b + 1 < nblk) vm_wait<kLoads>();
    else vm_wait<0>();
    const uint32_t t0 = b * FB;
    const int npc = static_cast<int>(((T - t0) < FB ? (T - t0) : FB) / 4);
    auto run_piece = [&](int pc, const Piece& x) __attribute__((always_inline)) {
      if (t0 + 4u * pc == next_ckpt) {
        st32(rbm, M, bm_off, ckpt * 32u);
        st32(rbc, P, bc_off, ckpt * 4u);
        ++ckpt;
        next_ckpt += chunk;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Hist h;
        step(P, M, x.k[j], x.d[j], x.p[j], x.r[j], x.v[j], a.floor, h);
        sl[S::V + 64 * (4 * pc + j) + lane] = fmaf(M, x.q[j], 0.f);
      }
    };
    if (npc == FB / 4) {
      // Whole block: unrolled, each piece's LDS reads issued two pieces
      // ahead into a ring of registers.
      constexpr int A = 2;  // pieces read ahead
      Piece x[A + 1];
#pragma unroll
      for (int pc = 0; pc < A; ++pc) read_piece<FB, FIXED>(sl, pc, seq, lane, true, true, x[pc]);
#pragma unroll
      for (int pc = 0; pc < FB / 4; ++pc) {
        if (pc + A < FB / 4) read_piece<FB, FIXED>(sl, pc + A, seq, lane, true, true, x[(pc + A) % (A + 1)]);
        run_piece(pc, x[pc % (A + 1)]);
      }
    } else {
      Piece cur;
      read_piece<FB, FIXED>(sl, 0, seq, lane, true, true, cur);
      for (int pc = 0; pc < npc; ++pc) {
        Piece nxt;
        read_piece<FB, FIXED>(sl, pc + 1 < npc ? pc + 1 : pc, seq, lane, true, true, nxt);
        run_piece(pc, cur);
        cur = nxt;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) st128<kNtSt>(ry, lds4(sl + S::V + 256 * i + 4 * lane), mp.v(i, t0, T), 0);
    if (b + kFwdSlots < nblk) issue(sl, t0 + kFwdSlots * FB);
  }
  st32(make_rsrc(a.mT + n0 * 8, valid * 32u), M, 4u * lane, 0);
  st32(make_rsrc(a.cT + n0, valid * 4u), P, col == 0 ? 4u * seq : kOob, 0);
  if (T > 0) {
    const uint32_t nb = static_cast<uint32_t>(a.nb);
    st32(rbm, M, bm_off, nb * 32u);
    st32(rbc, P, bc_off, nb * 4u);
  }
}

// Sum over the 8 lanes (value columns) of the caller's sequence.
__device__ __forceinline__ float colsum(float x) { return group_sum<8>(x); }

// Reverse of one token (the D = 1, one-column-per-lane case of reverse_step
// in bssm_step.h).  gM: own column of dL/dM; Gs: dL/dP (a symmetric scalar).
struct RevOut1 {
  float gk, gq, gd, gp, gr, gv;
};
template <bool DYN>
__device__ __forceinline__ void reverse(const Hist& h, float k, float d, float p, float q, float gy, float floor,
                                        float& gM, float& Gs, bool first, float& gc0, RevOut1& o) {
  const float beta = fast_rcp(fmaxf(h.s, floor));
  const float mp = d * h.M;
  const float Pb = fmaf(p, 1.f, (d * d) * h.P);
  const float bu = beta * h.u;
  const float gqp = fmaf(fmaf(bu, h.e, mp), gy, 0.f);
  gM = fmaf(q, gy, gM);
  const float ge = beta * fmaf(gM, h.u, 0.f);
  o.gv = ge;
  const float ap = fmaf(gM, h.e, 0.f);
  const float gkp = fmaf(-mp, ge, 0.f);
  const float gmb = fmaf(-k, ge, gM);
  const float gdp = DYN ? fmaf(gmb, h.M, 0.f) : 0.f;
  gM = gmb * d;
  const float av = colsum(ap);
  const float gkc = colsum(gkp);
  o.gq = colsum(gqp);
  const float gdc = DYN ? colsum(gdp) : 0.f;
  const float w = fmaf(Gs, h.u, 0.f);
  const float z = fmaf(h.u, av - w, 0.f);
  const float gs = (h.s > floor) ? -z * beta * beta : 0.f;
  const float gu = fmaf(beta, av - 2.f * w, gs * k);
  o.gk = fmaf(Pb, gu, fmaf(gs, h.u, gkc));
  const float dd = d * d;
  const float hsym = fmaf(0.5f, gu * k + gu * k, Gs);
  if (first) gc0 = fmaf(gu, k, Gs) * dd;
  Gs = hsym * dd;
  o.gd = DYN ? fmaf(2.f, fmaf(hsym * d, h.P, 0.f), gdc) : 0.f;
  o.gp = DYN ? hsym : 0.f;
  o.gr = DYN ? gs : 0.f;
}

template <bool FIXED, bool DYN>
__global__ __launch_bounds__(kWave) void backward_kernel(BwdArgs a) {
  __shared__ float tile[2 * kBwdSlot];
  using S = Slot<BB>;
  const int lane = threadIdx.x;
  const int seq = lane >> 3, col = lane & 7;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const uint32_t T = static_cast<uint32_t>(a.t);
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  const uint32_t row1 = T * 4u, row8 = T * 32u;
  const Rsrc rk = make_rsrc(a.k + n0 * T, valid * row1);
  const Rsrc rq = make_rsrc(a.q + n0 * T, valid * row1);
  const Rsrc rv = make_rsrc(a.v + n0 * T * 8, valid * row8);
  const Rsrc rgy = make_rsrc(a.gy + n0 * T * 8, valid * row8);
  const Rsrc rd = make_rsrc(FIXED ? a.k : a.d + n0 * T, FIXED ? 0u : valid * row1);
  const Rsrc rp = make_rsrc(FIXED ? a.k : a.p + n0 * T, FIXED ? 0u : valid * row1);
  const Rsrc rr = make_rsrc(FIXED ? a.k : a.r + n0 * T, FIXED ? 0u : valid * row1);
  const Rsrc rgk = make_rsrc(a.gk + n0 * T, valid * row1);
  const Rsrc rgq = make_rsrc(a.gq + n0 * T, valid * row1);
  const Rsrc rgv = make_rsrc(a.gv + n0 * T * 8, valid * row8);
  const Rsrc rgd = make_rsrc(a.gd ? a.gd + n0 * T : a.gk, a.gd ? valid * row1 : 0u);
  const Rsrc rgp = make_rsrc(a.gp ? a.gp + n0 * T : a.gk, a.gp ? valid * row1 : 0u);
  const Rsrc rgr = make_rsrc(a.gr ? a.gr + n0 * T : a.gk, a.gr ? valid * row1 : 0u);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 8, valid * nbp * 32u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp, valid * nbp * 4u);
  const Map mp(lane, row1, row8);
  const uint32_t bm_off = static_cast<uint32_t>(seq) * nbp * 32u + 4u * col;
  const uint32_t bc_off = static_cast<uint32_t>(seq) * nbp * 4u;

  // Carried adjoints: gM = dL/dM (own column), Gs = dL/dP (with one key
  // dimension sym(dL/dP) is dL/dP itself).
  float gM = a.gmf ? ld32(make_rsrc(a.gmf + n0 * 8, valid * 32u), 4u * lane, 0) : 0.f;
  float Gs = a.gcf ? ld32(make_rsrc(a.gcf + n0, valid * 4u), 4u * seq, 0) : 0.f;
  float gc0 = 0.f;

  const uint32_t nblk = (T + BB - 1) / BB;
  // Checkpoint beliefs of the two chunks of the next block to process.
  float nM[2], nP[2];
  auto issue = [&](float* sl, uint32_t b) __attribute__((always_inline)) {
    const uint32_t t0 = b * BB;
    const uint32_t off = mp.sc(0, t0, T);
    dma16<kNt>(rk, sl + S::K, off);
    dma16<kNt>(rq, sl + S::Q, off);
    if constexpr (!FIXED) {
      dma16<kNt>(rd, sl + S::D, off);
      dma16<kNt>(rp, sl + S::P, off);
      dma16<kNt>(rr, sl + S::R, off);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t ov = mp.v(i, t0, T);
      dma16<kNt>(rv, sl + S::V + 256 * i, ov);
      dma16<kNt>(rgy, sl + S::GY + 256 * i, ov);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t ck = 2u * b + h;
      const bool there = ck * kChunk < T;
      nM[h] = ld32(rbm, there ? bm_off + 32u * ck : kOob, 0);
      nP[h] = ld32(rbc, there ? bc_off + 4u * ck : kOob, 0);
    }
  };

  auto store_grads = [&](const float* sl, uint32_t b) __attribute__((always_inline)) {
    const uint32_t t0 = b * BB;
    const uint32_t off = mp.sc(0, t0, T);
    const int e = 4 * lane;
    st128<kNtSt>(rgk, lds4(sl + S::K + e), off, 0);
    st128<kNtSt>(rgq, lds4(sl + S::Q + e), off, 0);
    const v4f zero = v4f{0.f, 0.f, 0.f, 0.f};
    st128<kNtSt>(rgd, DYN ? lds4(sl + S::D + e) : zero, off, 0);
    st128<kNtSt>(rgp, DYN ? lds4(sl + S::P + e) : zero, off, 0);
    st128<kNtSt>(rgr, DYN ? lds4(sl + S::R + e) : zero, off, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) st128<kNtSt>(rgv, lds4(sl + S::V + 256 * i + e), mp.v(i, t0, T), 0);
  };

  // Replay one 16-token chunk (pieces pc0 .. pc0 + 3 of the slot) from its
  // checkpoint, then reverse it; the gradients overwrite the chunk's inputs.
  auto run_chunk = [&](float* sl, int pc0, float P, float M, bool first_chunk) __attribute__((always_inline)) {
    // The whole chunk's inputs are read up front: one LDS latency per chunk.
    Piece x[4];
    float gy[4][4];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      read_piece<BB, FIXED>(sl, pc0 + g4, seq, lane, true, true, x[g4]);
#pragma unroll
      for (int j = 0; j < 4; ++j) gy[g4][j] = sl[S::GY + 64 * (4 * (pc0 + g4) + j) + lane];
    }
    Hist h[kChunk];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        step(P, M, x[g4].k[j], x[g4].d[j], x[g4].p[j], x[g4].r[j], x[g4].v[j], a.floor, h[4 * g4 + j]);
#pragma unroll
    for (int g4 = 3; g4 >= 0; --g4) {
      const int pc = pc0 + g4;
      v4f gk, gq, gd, gp, gr;
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        RevOut1 o;
        reverse<DYN>(h[4 * g4 + j], x[g4].k[j], x[g4].d[j], x[g4].p[j], x[g4].q[j], gy[g4][j], a.floor, gM, Gs,
                     first_chunk && g4 == 0 && j == 0, gc0, o);
        gk[j] = o.gk;
        gq[j] = o.gq;
        gd[j] = o.gd;
        gp[j] = o.gp;
        gr[j] = o.gr;
        sl[S::V + 64 * (4 * pc + j) + lane] = o.gv;
      }
      if (col == 0) {
        const int o = 32 * pc + 4 * seq;
        lds4_store(sl + S::K + o, gk);
        lds4_store(sl + S::Q + o, gq);
        if constexpr (DYN) {
          lds4_store(sl + S::D + o, gd);
          lds4_store(sl + S::P + o, gp);
          lds4_store(sl + S::R + o, gr);
        }
      }
    }
  };

  // Block b is processed in slot b % 2.  At its start every outstanding
  // memory operation was issued a whole block earlier; then the gradients of
  // block b + 1 leave the other slot, which receives block b - 1.
  if (nblk > 0) issue(tile + ((nblk - 1) & 1) * kBwdSlot, nblk - 1);
  for (uint32_t i = 0; i < nblk; ++i) {
    const uint32_t b = nblk - 1 - i;
    float* cur = tile + (b & 1) * kBwdSlot;
    float* other = tile + ((b + 1) & 1) * kBwdSlot;
    vm_wait<0>();
    const float cM0 = nM[0], cM1 = nM[1], cP0 = nP[0], cP1 = nP[1];
    __syncthreads();
    if (b + 1 < nblk) store_grads(other, b + 1);
    if (b > 0) issue(other, b - 1);
    if ((2u * b + 1u) * kChunk < T) run_chunk(cur, 4, cP1, cM1, false);
    run_chunk(cur, 0, cP0, cM0, b == 0);
  }
  if (nblk > 0) {
    __syncthreads();
    store_grads(tile, 0);
  }
  if (a.gm0) st32(make_rsrc(a.gm0 + n0 * 8, valid * 32u), gM, 4u * lane, 0);
  if (a.gc0) st32(make_rsrc(a.gc0 + n0, valid * 4u), T > 0 ? gc0 : Gs, col == 0 ? 4u * seq : kOob, 0);
}

}  // namespace d1

bool d1_forward_ok(const FwdArgs& a) {
  return a.vec_kqd && a.vec_v && a.vec_pr && a.t % 4 == 0 && a.chunk % 4 == 0 && a.chunk < (int64_t(1) << 30) &&
         a.t * 256 < (int64_t(1) << 31) && (a.nb + 1) * 256 < (int64_t(1) << 31);
}

bool d1_backward_ok(const BwdArgs& a) {
  return a.vec_kqd && a.vec_v && a.vec_pr && a.t > 0 && a.t % d1::kChunk == 0 && a.chunk == d1::kChunk &&
         a.t * 256 < (int64_t(1) << 31) && (a.nb + 1) * 256 < (int64_t(1) << 31);
}

hipError_t launch_forward_d1(bool fixed, const FwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + d1::SPW - 1) / d1::SPW;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  if (fixed) hipLaunchKernelGGL((d1::forward_kernel<true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((d1::forward_kernel<false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_backward_d1(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + d1::SPW - 1) / d1::SPW;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  if (fixed) hipLaunchKernelGGL((d1::backward_kernel<true, false>), grid, block, 0, stream, a);
  else if (dyn) hipLaunchKernelGGL((d1::backward_kernel<false, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((d1::backward_kernel<false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace bssm
