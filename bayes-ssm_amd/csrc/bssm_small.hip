// Row-per-sequence kernels for D = 4, M = 8 at small sequence counts, gfx950.
//
// The rotated-layout kernels (bssm_rot4.h) give a quad of 4 lanes to each
// sequence, 16 sequences per wave.  Below about 1024 x 16 sequences their
// waves do not fill the SIMDs, and each wave's time is its own instruction
// stream: a wave issues the same instructions whatever number of its lanes
// hold live sequences.  Here a 16-lane DPP row holds one sequence (4 per
// wave) and every lane one entry of the covariance, so the per-token stream
// is about 40 % shorter (four times as many waves, each doing a quarter of
// the state).  The row layout spends about 2.4 times the lane work per
// sequence, so once every SIMD holds several waves the rotated layout wins:
// for the backward above about 8192 sequences, for the forward (which at
// 16384 sequences still gains from its 4 waves per SIMD against the rotated
// layout's one) above about 24576.
//
// Lane (i, j) of a sequence's row (i = row bits 3:2, j = bits 1:0) holds
//   P[i][j]                    (the covariance, bitwise symmetric)
//   M[j][2i], M[j][2i + 1]     (the mean, transposed: row j of M)
// The forward keeps the lane's mean pair in its own order instead,
// (M[j][c], M[j][c ^ 1]) with c = 2i + (j & 1): the lanes j, j ^ 1 of a quad
// then hold the same column pair in opposite order, so a sum over j of a
// column is an exchange between them and one quad step that leaves each lane
// its own column's sum (and its partner the other's): a reduce-scatter in
// place of two all-reduces for the readout and the innovations.  In the
// backward the extra exchange lengthens the chained reverse; it keeps the
// record order.
// Sums over j are quad all-reduces (xor 1, xor 2); sums over i are
// "column" all-reduces over the row: the pair (i, i ^ 1) through the half-row
// mirror and a quad reversal, then the pairs through a row rotation by 8.
// Both pair their four terms as ((a0 + a1) + (a2 + a3)), so a row sum and the
// matching column sum of the symmetric covariance give the same bits, and
// every quantity a lane needs in both orientations (u_i and u_j) is formed
// from them identically: the covariance update stays bitwise symmetric.
//
// The equations are those of bssm_rot4.h (forward_step): u = d * (P (d * k))
// + p k, s = r + k.u, beta = 1 / max(s, floor), e = v - (d * M)^T k,
// M <- d * M + beta u e^T, P <- d d^T * P + p I - beta u u^T, y = M^T q.

#include <atomic>
#include <cfloat>

#include "bssm_rot4.h"

// No contraction: a sum like x + dpp(x) with x = a * b would otherwise be
// fused into fma(a, b, dpp(x)), which rounds the two lanes of a pair
// differently and breaks the bitwise agreement of row and column sums.
// Every intended fused multiply-add is an explicit fmaf.
#pragma clang fp contract(off)

namespace bssm {
namespace sn {
namespace {

constexpr int SPW = 4;   // sequences per wave
constexpr int TT = 16;   // tokens per staged tile
constexpr int kRowRor8 = 0x128;
constexpr int kQuadRev = quad_perm(3, 2, 1, 0);

using r4::Rsrc;
using r4::make_rsrc;
using r4::kOob;
using r4::v4u;
typedef float v2f __attribute__((ext_vector_type(2)));

// Sum over the 4 lanes j of the quad; identical bits in the quad.
__device__ __forceinline__ float quad_sum(float x) {
  x += dpp<kXor1>(x);
  return x + dpp<kXor2>(x);
}
// Sum over the 4 rows i of the 16-lane row at fixed j; identical bits in the
// column, and equal to quad_sum of the transposed terms.
__device__ __forceinline__ float col_sum(float x) {
  const float m = dpp<kHalfMirror>(x);  // lane (i ^ 1, 3 - j)
  x += dpp<kQuadRev>(m);                // + lane (i ^ 1, j)
  return x + dpp<kRowRor8>(x);          // + rows i ^ 2, i ^ 3
}

// LDS tile of one wave: per sequence k, d, q [TT][4], v / y [TT][8], p, r
// [TT], at a stride of 8 banks (mod 32), so that the 4 sequences' reads of
// one token (4 key or 8 value words each) fall in different banks.
struct Tile {
  static constexpr int K = 0, D = 64, Q = 128, V = 192, P = 320, R = 336, SEQ = 360, SIZE = SPW * SEQ;
};

// Register staging of one tile: lane (s, c) (s = lane >> 4, c = lane & 15)
// loads token c's 16-byte k / d / q piece of sequence s, v pieces c and
// c + 16 (token piece >> 1, half piece & 1), and for c < 4 the p / r piece c
// (tokens 4c .. 4c + 3).
struct Stage {
  v4f k, d, q, v0, v1, p, r;
};

// Keys, queries and values may arrive as bfloat16 or float8 (F, an InFmt);
// they are widened exactly to float32 as they are written to LDS, so the
// kernels' arithmetic is the float32 one on the widened values.  Bytes per
// token of a 4-value stream (k, q) in format F; a value row takes twice that.
template <int F>
constexpr uint32_t kq_bytes() {
  return F == kInF32 ? 16u : F == kInBf16 ? 8u : 4u;
}
// Lanes (of a sequence's 16) that move the 16-byte pieces of a 4-value
// stream over TOK tokens; a value stream takes twice as many pieces (float32
// at 16 tokens: two per lane, c and c + 16).
template <int F, int TOK = TT>
constexpr int kq_lanes() {
  return static_cast<int>(TOK * kq_bytes<F>() / 16u);
}

// Raw 16-byte pieces (lane c of sequence s) of the TOK tokens from t0 of the
// 4-value stream r, and of the value stream rv (two pieces for float32 at 16
// tokens).
template <int F, int TOK = TT>
__device__ __forceinline__ v4f load_kq(Rsrc r, uint32_t row, int s, int c, uint32_t t0) {
  const uint32_t off = static_cast<uint32_t>(s) * row + t0 * kq_bytes<F>() + static_cast<uint32_t>(c) * 16u;
  return r4::ld128<true>(r, c < kq_lanes<F, TOK>() ? off : kOob);
}
template <int F, int TOK = TT>
__device__ __forceinline__ void load_v(v4f& v0, v4f& v1, Rsrc rv, uint32_t row, int s, int c, uint32_t t0) {
  const uint32_t off = static_cast<uint32_t>(s) * row + t0 * 2u * kq_bytes<F>() + static_cast<uint32_t>(c) * 16u;
  v0 = r4::ld128<true>(rv, c < 2 * kq_lanes<F, TOK>() ? off : kOob);
  if constexpr (F == kInF32 && TOK == 16) v1 = r4::ld128<true>(rv, off + 256u);
}
// Widen and write those pieces into a tile region of TOK x 4 (k, q) or TOK x 8
// (v) floats.
template <int F, int TOK = TT>
__device__ __forceinline__ void put_kq(float* dst, v4f x, int c) {
  if (c >= kq_lanes<F, TOK>()) return;
  if constexpr (F == kInF32) {
    *reinterpret_cast<v4f*>(dst + 4 * c) = x;
  } else if constexpr (F == kInBf16) {  // tokens 2c, 2c + 1
    *reinterpret_cast<v4f*>(dst + 8 * c) = r4::widen_lo(x);
    *reinterpret_cast<v4f*>(dst + 8 * c + 4) = r4::widen_hi(x);
  } else {  // tokens 4c .. 4c + 3, one 32-bit word each
    const v4u w = __builtin_bit_cast(v4u, x);
#pragma unroll
    for (int u = 0; u < 4; ++u) *reinterpret_cast<v4f*>(dst + 16 * c + 4 * u) = widen_f8<F>(w[u]);
  }
}
template <int F, int TOK = TT>
__device__ __forceinline__ void put_v(float* dst, v4f v0, v4f v1, int c) {
  if constexpr (F == kInF32 && TOK == 16) {  // pieces c and c + 16 (token piece >> 1, half piece & 1)
    *reinterpret_cast<v4f*>(dst + 4 * c) = v0;
    *reinterpret_cast<v4f*>(dst + 64 + 4 * c) = v1;
  } else {
    if (c >= 2 * kq_lanes<F, TOK>()) return;
    if constexpr (F == kInF32) {  // piece c
      *reinterpret_cast<v4f*>(dst + 4 * c) = v0;
    } else if constexpr (F == kInBf16) {  // token c
      *reinterpret_cast<v4f*>(dst + 8 * c) = r4::widen_lo(v0);
      *reinterpret_cast<v4f*>(dst + 8 * c + 4) = r4::widen_hi(v0);
    } else {  // tokens 2c, 2c + 1, half a token per word
      const v4u w = __builtin_bit_cast(v4u, v0);
#pragma unroll
      for (int u = 0; u < 4; ++u) *reinterpret_cast<v4f*>(dst + 16 * c + 4 * u) = widen_f8<F>(w[u]);
    }
  }
}
// The reverse: gradients in a region of TOK x 4 / TOK x 8 floats leave as
// 16-byte pieces of format F (bfloat16: round to nearest even; float8:
// narrow_f8, torch's rounding), at the loaders' offsets.
template <int F, int TOK>
__device__ __forceinline__ void store_kq(Rsrc r, uint32_t row, int s, int c, uint32_t t0, const float* src) {
  const uint32_t off = static_cast<uint32_t>(s) * row + t0 * kq_bytes<F>() + static_cast<uint32_t>(c) * 16u;
  const uint32_t o = c < kq_lanes<F, TOK>() ? off : kOob;
  const int cc = c & (kq_lanes<F, TOK>() - 1);
  v4f x;
  if constexpr (F == kInF32) {
    x = *reinterpret_cast<const v4f*>(src + 4 * cc);
  } else if constexpr (F == kInBf16) {
    x = r4::narrow(*reinterpret_cast<const v4f*>(src + 8 * cc), *reinterpret_cast<const v4f*>(src + 8 * cc + 4));
  } else {
    v4u w;
#pragma unroll
    for (int u = 0; u < 4; ++u) w[u] = narrow_f8<F>(*reinterpret_cast<const v4f*>(src + 16 * cc + 4 * u));
    x = __builtin_bit_cast(v4f, w);
  }
  r4::st128<r4::kNtStore>(r, x, o, 0);
}
template <int F, int TOK>
__device__ __forceinline__ void store_v(Rsrc r, uint32_t row, int s, int c, uint32_t t0, const float* src) {
  static_assert(TOK * 2 * kq_bytes<F>() <= 256u, "one piece per lane");
  const uint32_t off = static_cast<uint32_t>(s) * row + t0 * 2u * kq_bytes<F>() + static_cast<uint32_t>(c) * 16u;
  const int lanes = 2 * kq_lanes<F, TOK>();
  const uint32_t o = c < lanes ? off : kOob;
  const int cc = c & (lanes - 1);
  v4f x;
  if constexpr (F == kInF32) {
    x = *reinterpret_cast<const v4f*>(src + 4 * cc);
  } else if constexpr (F == kInBf16) {
    x = r4::narrow(*reinterpret_cast<const v4f*>(src + 8 * cc), *reinterpret_cast<const v4f*>(src + 8 * cc + 4));
  } else {
    v4u w;
#pragma unroll
    for (int u = 0; u < 4; ++u) w[u] = narrow_f8<F>(*reinterpret_cast<const v4f*>(src + 16 * cc + 4 * u));
    x = __builtin_bit_cast(v4f, w);
  }
  r4::st128<r4::kNtStore>(r, x, o, 0);
}

struct Streams {
  Rsrc k, d, q, v, p, r, y;
  uint32_t row4, row8, row1;    // float32 bytes per sequence row
  uint32_t row4n, row8n;        // bytes per sequence row of k, q and of v in their format
};

template <bool FIXED, int F>
__device__ __forceinline__ void load_tile(Stage& x, const Streams& st, int s, int c, uint32_t t0) {
  const uint32_t o4 = static_cast<uint32_t>(s) * st.row4 + (t0 + c) * 16u;
  x.k = load_kq<F>(st.k, st.row4n, s, c, t0);
  x.q = load_kq<F>(st.q, st.row4n, s, c, t0);
  if constexpr (!FIXED) x.d = r4::ld128<true>(st.d, o4);
  load_v<F>(x.v0, x.v1, st.v, st.row8n, s, c, t0);
  if constexpr (!FIXED) {
    const uint32_t o1 = c < 4 ? static_cast<uint32_t>(s) * st.row1 + t0 * 4u + c * 16u : kOob;
    x.p = r4::ld128<false>(st.p, o1);
    x.r = r4::ld128<false>(st.r, o1);
  }
}

template <bool FIXED, int F>
__device__ __forceinline__ void put_tile(const Stage& x, float* tl, int s, int c) {
  float* b = tl + s * Tile::SEQ;
  put_kq<F>(b + Tile::K, x.k, c);
  put_kq<F>(b + Tile::Q, x.q, c);
  put_v<F>(b + Tile::V, x.v0, x.v1, c);
  if constexpr (!FIXED) {
    *reinterpret_cast<v4f*>(b + Tile::D + 4 * c) = x.d;
    if (c < 4) {
      *reinterpret_cast<v4f*>(b + Tile::P + 4 * c) = x.p;
      *reinterpret_cast<v4f*>(b + Tile::R + 4 * c) = x.r;
    }
  }
}

// Token inputs of lane (i, j).
struct Tok {
  float ki, kj, di, dj, qj, p, r;
  v2f v;  // v[2i], v[2i + 1]; in the forward's own order v[c], v[c ^ 1]
};

template <bool FIXED>
__device__ __forceinline__ void read_tok(Tok& x, const float* b, int tt, int i, int j) {
  x.ki = b[Tile::K + 4 * tt + i];
  x.kj = b[Tile::K + 4 * tt + j];
  x.qj = b[Tile::Q + 4 * tt + j];
  const int co = 2 * i + (j & 1);
  x.v[0] = b[Tile::V + 8 * tt + co];
  x.v[1] = b[Tile::V + 8 * tt + (co ^ 1)];
  if constexpr (FIXED) {
    x.di = x.dj = kFixedDecay;
    x.p = kFixedProcess;
    x.r = kFixedObservation;
  } else {
    x.di = b[Tile::D + 4 * tt + i];
    x.dj = b[Tile::D + 4 * tt + j];
    x.p = b[Tile::P + tt];
    x.r = b[Tile::R + tt];
  }
}

// Belief of lane (i, j) and its step.
struct Bel {
  float P, M0, M1;
};

// The lane's mean pair between record order (columns 2i, 2i + 1) and its own
// order (c, c ^ 1); the same swap both ways.
__device__ __forceinline__ v2f own_order(v2f m, bool odd) {
  v2f r;
  r[0] = odd ? m[1] : m[0];
  r[1] = odd ? m[0] : m[1];
  return r;
}

// Sum over the quad of the lane's own column, given the lane's terms of its
// own column (x0) and of the other (x1).
__device__ __forceinline__ float own_sum(float x0, float x1) {
  const float t = x0 + dpp<kXor1>(x1);
  return t + dpp<kXor2>(t);
}

struct StepOut {
  float ui, uj, s;
  v2f e;
};

// OWN: mean pair, values and innovations in the lane's own order.  TR: u_j
// is read from the transposed lane (j, i) of the sequence (byte address tr
// for ds_bpermute), whose u_i has the same bits as the column sum gives (P
// is bitwise symmetric and col_sum pairs its terms as quad_sum does): one LDS
// crossbar instruction in place of six VALU instructions.
template <bool OWN, bool TR = false>
__device__ __forceinline__ void forward_step(Bel& b, const Tok& x, float delta, float floor, StepOut& o,
                                             int tr = 0) {
  const float wkj = x.dj * x.kj;
  const float zi = quad_sum(b.P * wkj);  // (P (d * k))_i
  const float ui = fmaf(x.di, zi, x.p * x.ki);
  float uj;
  if constexpr (TR) {
    uj = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(tr, __builtin_bit_cast(int, ui)));
  } else {
    const float zj = col_sum(b.P * (x.di * x.ki));  // (P (d * k))_j, the same bits for i == j
    uj = fmaf(x.dj, zj, x.p * x.kj);
  }
  const float s = quad_sum(x.kj * uj) + x.r;
  const float beta = fast_rcp(fmaxf(s, floor));
  // Innovations of the lane's two columns: e = v - sum_j M[j][.] d_j k_j (in
  // own order the other column's sum is the partner's own).
  float e0, e1;
  if constexpr (OWN) {
    const float so = own_sum(b.M0 * wkj, b.M1 * wkj);
    e0 = x.v[0] - so;
    e1 = x.v[1] - dpp<kXor1>(so);
  } else {
    e0 = x.v[0] - quad_sum(b.M0 * wkj);
    e1 = x.v[1] - quad_sum(b.M1 * wkj);
  }
  const float bu = beta * uj;
  b.M0 = fmaf(bu, e0, x.dj * b.M0);
  b.M1 = fmaf(bu, e1, x.dj * b.M1);
  const float dp = fmaf(x.p, delta, (x.di * x.dj) * b.P);
  b.P = fmaf(-beta, ui * uj, dp);
  o.ui = ui;
  o.uj = uj;
  o.s = s;
  o.e[0] = e0;
  o.e[1] = e1;
}

// Readout of the lane's own column after the token (own order):
// y_c = sum_j M[j][c] q_j.
__device__ __forceinline__ float readout(const Bel& b, float qj) { return own_sum(b.M0 * qj, b.M1 * qj); }

// Belief record offsets of lane (i, j) (bytes within one sequence's record).
__device__ __forceinline__ uint32_t mean_off(int i, int j) { return static_cast<uint32_t>(j * 32 + i * 8); }
__device__ __forceinline__ uint32_t cov_off(int i, int j) { return static_cast<uint32_t>(i * 16 + j * 4); }

template <bool FIXED, int F>
__global__ __launch_bounds__(kWave) void forward_kernel(FwdArgs a) {
  __shared__ float tile[Tile::SIZE];
  const int lane = threadIdx.x;
  const int s = lane >> 4, c = lane & 15, i = c >> 2, j = c & 3;
  const int co = 2 * i + (j & 1);  // the lane's own value column
  const int tr = 4 * (16 * s + 4 * j + i);  // ds_bpermute address of lane (j, i)
  const bool odd = (j & 1) != 0;
  const float delta = i == j ? 1.f : 0.f;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t T = a.t;
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  Streams st;
  st.row4 = static_cast<uint32_t>(T) * 16u;
  st.row8 = static_cast<uint32_t>(T) * 32u;
  st.row1 = static_cast<uint32_t>(T) * 4u;
  st.row4n = static_cast<uint32_t>(T) * kq_bytes<F>();
  st.row8n = 2u * st.row4n;
  st.k = make_rsrc(r4::byte_offset(a.k, n0 * st.row4n), valid * st.row4n);
  st.q = make_rsrc(r4::byte_offset(a.q, n0 * st.row4n), valid * st.row4n);
  st.v = make_rsrc(r4::byte_offset(a.v, n0 * st.row8n), valid * st.row8n);
  st.y = make_rsrc(a.y + n0 * T * 8, valid * st.row8);
  st.d = make_rsrc(FIXED ? a.y : a.d + n0 * T * 4, FIXED ? 0u : valid * st.row4);
  st.p = make_rsrc(FIXED ? a.k : a.p + n0 * T, FIXED ? 0u : valid * st.row1);
  st.r = make_rsrc(FIXED ? a.k : a.r + n0 * T, FIXED ? 0u : valid * st.row1);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 32, valid * nbp * 128u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 16, valid * nbp * 64u);
  const Rsrc rm0 = make_rsrc(a.m0 + n0 * 32, valid * 128u);
  const Rsrc rc0 = make_rsrc(a.c0 + n0 * 16, valid * 64u);
  const Rsrc rmT = make_rsrc(a.mT + n0 * 32, valid * 128u);
  const Rsrc rcT = make_rsrc(a.cT + n0 * 16, valid * 64u);
  // Lane offsets in the belief records: the state tensors hold one record per
  // sequence, the checkpoints nb + 1.
  const uint32_t mo = static_cast<uint32_t>(s) * 128u + mean_off(i, j), cvo = static_cast<uint32_t>(s) * 64u + cov_off(i, j);
  const uint32_t cmo = static_cast<uint32_t>(s) * nbp * 128u + mean_off(i, j),
                 cco = static_cast<uint32_t>(s) * nbp * 64u + cov_off(i, j);

  Bel b;
  {
    const v2f m = own_order(r4::ld64(rm0, mo, 0), odd);
    b.M0 = m[0];
    b.M1 = m[1];
    b.P = r4::ld32(rc0, cvo, 0);
  }
  // The initial belief has landed before the loop (a load pending at the
  // loop header would make every iteration wait for all outstanding loads).
  r4::vm_wait<0>();
  auto store_ckpt = [&](uint32_t rec) __attribute__((always_inline)) {
    v2f m;
    m[0] = b.M0;
    m[1] = b.M1;
    r4::st64(rbm, own_order(m, odd), cmo, rec * 128u);
    r4::st32(rbc, b.P, cco, rec * 64u);
  };
  store_ckpt(0);

  float* mine = tile + s * Tile::SEQ;
  const int64_t ntiles = (T + TT - 1) / TT;
  Stage x;
  if (ntiles > 0) load_tile<FIXED, F>(x, st, s, c, 0);
  int64_t next_ckpt = a.chunk;
  uint32_t ckpt = 1;
  v4f ys0 = v4f{0.f, 0.f, 0.f, 0.f}, ys1 = ys0;
  for (int64_t ti = 0; ti < ntiles; ++ti) {
    const uint32_t t0 = static_cast<uint32_t>(ti * TT);
    const int len = static_cast<int>((T - t0) < TT ? (T - t0) : TT);
    // The previous tile's readouts leave LDS before this tile lands there.
    if (ti > 0) {
      ys0 = *reinterpret_cast<const v4f*>(mine + Tile::V + 4 * c);
      ys1 = *reinterpret_cast<const v4f*>(mine + Tile::V + 64 + 4 * c);
    }
    r4::vm_wait<0>();
    put_tile<FIXED, F>(x, tile, s, c);
    if (ti > 0) {
      // Pieces c (token c >> 1) and c + 16 of the previous tile, all of whose tokens were computed.
      const uint32_t p0 = t0 - TT, o8 = static_cast<uint32_t>(s) * st.row8 + p0 * 32u + c * 16u;
      r4::st128<r4::kNtStore>(st.y, ys0, o8, 0);
      r4::st128<r4::kNtStore>(st.y, ys1, o8 + 256u, 0);
    }
    if (ti + 1 < ntiles) load_tile<FIXED, F>(x, st, s, c, t0 + TT);
    r4::lds_wait();
    if (len == TT && a.chunk % 8 == 0) {
#pragma unroll
      for (int h = 0; h < TT / 8; ++h) {
        if (static_cast<int64_t>(t0) + 8 * h == next_ckpt) {
          store_ckpt(ckpt++);
          next_ckpt += a.chunk;
        }
        Tok cur, nxt;
        read_tok<FIXED>(cur, mine, 8 * h, i, j);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int tt = 8 * h + u;
          if (u + 1 < 8) read_tok<FIXED>(nxt, mine, tt + 1, i, j);
          StepOut o;
          forward_step<true, true>(b, cur, delta, a.floor, o, tr);
          mine[Tile::V + 8 * tt + co] = readout(b, cur.qj);
          cur = nxt;
        }
      }
    } else {
      for (int tt = 0; tt < len; ++tt) {
        if (static_cast<int64_t>(t0) + tt == next_ckpt) {
          store_ckpt(ckpt++);
          next_ckpt += a.chunk;
        }
        Tok cur;
        read_tok<FIXED>(cur, mine, tt, i, j);
        StepOut o;
        forward_step<true, true>(b, cur, delta, a.floor, o, tr);
        mine[Tile::V + 8 * tt + co] = readout(b, cur.qj);
      }
    }
  }
  if (ntiles > 0) {
    // The last tile's readouts: only the pieces of its valid tokens.
    const uint32_t t0 = static_cast<uint32_t>((ntiles - 1) * TT);
    const int len = static_cast<int>(T - t0);
    r4::lds_wait();
    ys0 = *reinterpret_cast<const v4f*>(mine + Tile::V + 4 * c);
    ys1 = *reinterpret_cast<const v4f*>(mine + Tile::V + 64 + 4 * c);
    const uint32_t o8 = static_cast<uint32_t>(s) * st.row8 + t0 * 32u + c * 16u;
    r4::st128<r4::kNtStore>(st.y, ys0, (c >> 1) < len ? o8 : kOob, 0);
    r4::st128<r4::kNtStore>(st.y, ys1, ((c + 16) >> 1) < len ? o8 + 256u : kOob, 0);
  }
  v2f m;
  m[0] = b.M0;
  m[1] = b.M1;
  r4::st64(rmT, own_order(m, odd), mo, 0);
  r4::st32(rcT, b.P, cvo, 0);
  store_ckpt(static_cast<uint32_t>(a.nb));
}

// ------------------------------------------------- two-wave forward (split)
// At the smallest sequence counts the single-wave kernels leave SIMDs idle,
// and each wave's time is its instruction stream.  The step splits into a
// covariance half and a mean half that only talk one way: the mean update
// needs the gain column bu_j = beta u_j, nothing else of the covariance
// chain.  Here a workgroup of two waves holds the same 4 sequences: wave 0
// runs the covariance chain (u, s, beta, P) one 16-token tile ahead and
// leaves bu in LDS; wave 1 runs the innovations, the mean update and the
// readouts of the tile before, from those bu.  One barrier per tile; each
// wave stages and stores its own streams (wave 0: k, d, p, r, the covariance
// checkpoints and final covariance; wave 1: v, q, the readouts, the mean
// checkpoints and final mean).  The operations are those of forward_step, in
// the same order, so the results are bitwise those of forward_kernel.
struct STile {
  // Input slot per sequence (3 slots: tile t + 1 lands while tiles t and
  // t - 1 are read): k, d, q [TT][4], v [TT][8], p, r [TT].
  static constexpr int K = 0, D = 64, Q = 128, V = 192, P = 320, R = 336, SEQ = 360, SLOT = SPW * SEQ;
  // Readouts of a tile (2 slots) and the gain columns bu (2 slots).
  static constexpr int YSEQ = 136, YSLOT = SPW * YSEQ, BSEQ = 72, BSLOT = SPW * BSEQ;
  static constexpr int IN = 0, Y = 3 * SLOT, BU = Y + 2 * YSLOT, SIZE = BU + 2 * BSLOT;
};

// Covariance half of forward_step: P advanced, the gain column bu_j returned.
__device__ __forceinline__ float cov_step(float& P, float ki, float kj, float di, float dj, float p, float r,
                                          float delta, float floor) {
  const float wki = di * ki, wkj = dj * kj;
  const float zi = quad_sum(P * wkj);
  const float zj = col_sum(P * wki);
  const float ui = fmaf(di, zi, p * ki), uj = fmaf(dj, zj, p * kj);
  const float s = quad_sum(kj * uj) + r;
  const float beta = fast_rcp(fmaxf(s, floor));
  const float bu = beta * uj;
  const float dp = fmaf(p, delta, (di * dj) * P);
  P = fmaf(-beta, ui * uj, dp);
  return bu;
}

// Mean half (own order) and the readout of the lane's own column.
__device__ __forceinline__ float mean_step(float& M0, float& M1, float kj, float dj, float qj, v2f v, float bu) {
  const float wkj = dj * kj;
  const float so = own_sum(M0 * wkj, M1 * wkj);
  const float e0 = v[0] - so;
  const float e1 = v[1] - dpp<kXor1>(so);
  M0 = fmaf(bu, e0, dj * M0);
  M1 = fmaf(bu, e1, dj * M1);
  return own_sum(M0 * qj, M1 * qj);
}

// G groups of SPW sequences per workgroup, two waves each (covariance A, B,
// then mean A, B): with G = 2 the four waves take the CU's four SIMDs, where
// two two-wave workgroups on one CU leave a SIMD idle and make two waves share
// one (the hardware places a workgroup's waves in the cyclic SIMD order 0, 2,
// 1, 3 and starts the next workgroup at the previous one's second SIMD).
template <bool FIXED, int F, int G>
__global__ __launch_bounds__(2 * G * kWave) void forward_split_kernel(FwdArgs a) {
  __shared__ float lds_all[G * STile::SIZE];
  // The wave index, uniform across the wave (so are the group and its
  // addresses and buffer descriptors).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const bool cov_wave = G == 1 ? wave == 0 : wave < 2;
  const int grp = G == 1 ? 0 : (wave & 1);
  float* const lds = lds_all + grp * STile::SIZE;
  const int s = lane >> 4, c = lane & 15, i = c >> 2, j = c & 3;
  const int co = 2 * i + (j & 1);
  const bool odd = (j & 1) != 0;
  const float delta = i == j ? 1.f : 0.f;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * G + grp) * SPW;
  const int64_t T = a.t;
  const int64_t rest = a.n - n0;  // the last workgroup's second group may hold none
  const uint32_t valid = static_cast<uint32_t>(rest <= 0 ? 0 : rest < SPW ? rest : SPW);
  const uint32_t row4 = static_cast<uint32_t>(T) * 16u, row8 = static_cast<uint32_t>(T) * 32u,
                 row1 = static_cast<uint32_t>(T) * 4u;
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  // Tile indices in 32-bit arithmetic (T * 32 bytes fits a descriptor's range).
  const uint32_t T32 = static_cast<uint32_t>(T);
  const uint32_t ntiles = (T32 + TT - 1) / TT;
  auto in_slot = [&](uint32_t t) __attribute__((always_inline)) {
    return lds + STile::IN + static_cast<int>(t % 3u) * STile::SLOT + s * STile::SEQ;
  };
  auto y_slot = [&](uint32_t t) __attribute__((always_inline)) {
    return lds + STile::Y + static_cast<int>(t & 1u) * STile::YSLOT + s * STile::YSEQ;
  };
  auto bu_slot = [&](uint32_t t) __attribute__((always_inline)) {
    return lds + STile::BU + static_cast<int>(t & 1u) * STile::BSLOT + s * STile::BSEQ;
  };
  auto tile_len = [&](uint32_t t) __attribute__((always_inline)) {
    return static_cast<int>((T32 - t * TT) < TT ? (T32 - t * TT) : TT);
  };

  if (cov_wave) {
    // ---- covariance wave
    const uint32_t row4n = static_cast<uint32_t>(T) * kq_bytes<F>();
    const Rsrc rk = make_rsrc(r4::byte_offset(a.k, n0 * row4n), valid * row4n);
    const Rsrc rd = make_rsrc(FIXED ? a.k : a.d + n0 * T * 4, FIXED ? 0u : valid * row4);
    const Rsrc rp = make_rsrc(FIXED ? a.k : a.p + n0 * T, FIXED ? 0u : valid * row1);
    const Rsrc rr = make_rsrc(FIXED ? a.k : a.r + n0 * T, FIXED ? 0u : valid * row1);
    const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 16, valid * nbp * 64u);
    const Rsrc rc0 = make_rsrc(a.c0 + n0 * 16, valid * 64u);
    const Rsrc rcT = make_rsrc(a.cT + n0 * 16, valid * 64u);
    const uint32_t cvo = static_cast<uint32_t>(s) * 64u + cov_off(i, j);
    const uint32_t cco = static_cast<uint32_t>(s) * nbp * 64u + cov_off(i, j);
    v4f sk, sd, sp, sr;
    auto load = [&](uint32_t t) __attribute__((always_inline)) {
      const uint32_t t0 = t * TT;
      const uint32_t o4 = static_cast<uint32_t>(s) * row4 + (t0 + c) * 16u;
      sk = load_kq<F>(rk, row4n, s, c, t0);
      if constexpr (!FIXED) {
        sd = r4::ld128<true>(rd, o4);
        const uint32_t o1 = c < 4 ? static_cast<uint32_t>(s) * row1 + t0 * 4u + c * 16u : kOob;
        sp = r4::ld128<false>(rp, o1);
        sr = r4::ld128<false>(rr, o1);
      }
    };
    auto put = [&](uint32_t t) __attribute__((always_inline)) {
      float* b = in_slot(t);
      put_kq<F>(b + STile::K, sk, c);
      if constexpr (!FIXED) {
        *reinterpret_cast<v4f*>(b + STile::D + 4 * c) = sd;
        if (c < 4) {
          *reinterpret_cast<v4f*>(b + STile::P + 4 * c) = sp;
          *reinterpret_cast<v4f*>(b + STile::R + 4 * c) = sr;
        }
      }
    };
    float P = r4::ld32(rc0, cvo, 0);
    r4::vm_wait<0>();
    r4::st32(rbc, P, cco, 0);
    if (ntiles > 0) {
      load(0);
      r4::vm_wait<0>();
      put(0);
      if (ntiles > 1) load(1);
    }
    __syncthreads();
    int64_t next_ckpt = a.chunk;
    uint32_t ckpt = 1;
    for (uint32_t it = 0; it <= ntiles; ++it) {
      if (it + 1 < ntiles) {
        r4::vm_wait<0>();
        put(it + 1);
        if (it + 2 < ntiles) load(it + 2);
      }
      if (it < ntiles) {
        const float* b = in_slot(it);
        float* bu = bu_slot(it);
        const int64_t t0 = it * TT;
        const int len = tile_len(it);
        // Each token's inputs are read one token ahead, before the previous
        // token's bu write (LDS reads may not pass that write).
        struct In {
          float ki, kj, di, dj, p, r;
        };
        auto read = [&](In& x, int tt) __attribute__((always_inline)) {
          x.ki = b[STile::K + 4 * tt + i];
          x.kj = b[STile::K + 4 * tt + j];
          x.di = FIXED ? kFixedDecay : b[STile::D + 4 * tt + i];
          x.dj = FIXED ? kFixedDecay : b[STile::D + 4 * tt + j];
          x.p = FIXED ? kFixedProcess : b[STile::P + tt];
          x.r = FIXED ? kFixedObservation : b[STile::R + tt];
        };
        auto ckpt_at = [&](int64_t t) __attribute__((always_inline)) {
          if (t == next_ckpt) {
            r4::st32(rbc, P, cco, ckpt * 64u);
            ++ckpt;
            next_ckpt += a.chunk;
          }
        };
        In cur, nxt;
        read(cur, 0);
        if (len == TT && a.chunk % 8 == 0) {
          // Checkpoints can only fall on tokens 0 and 8 of a full tile: two
          // straight 8-token runs.
#pragma unroll
          for (int h = 0; h < TT / 8; ++h) {
            ckpt_at(t0 + 8 * h);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              const int tt = 8 * h + u;
              if (tt + 1 < TT) read(nxt, tt + 1);
              bu[4 * tt + j] = cov_step(P, cur.ki, cur.kj, cur.di, cur.dj, cur.p, cur.r, delta, a.floor);
              cur = nxt;
            }
          }
        } else {
          for (int tt = 0; tt < len; ++tt) {
            if (tt + 1 < len) read(nxt, tt + 1);
            ckpt_at(t0 + tt);
            bu[4 * tt + j] = cov_step(P, cur.ki, cur.kj, cur.di, cur.dj, cur.p, cur.r, delta, a.floor);
            cur = nxt;
          }
        }
      }
      __syncthreads();
    }
    r4::st32(rcT, P, cvo, 0);
    r4::st32(rbc, P, cco, static_cast<uint32_t>(a.nb) * 64u);
  } else {
    // ---- mean wave
    const uint32_t row4n = static_cast<uint32_t>(T) * kq_bytes<F>(), row8n = 2u * row4n;
    const Rsrc rq = make_rsrc(r4::byte_offset(a.q, n0 * row4n), valid * row4n);
    const Rsrc rv = make_rsrc(r4::byte_offset(a.v, n0 * row8n), valid * row8n);
    const Rsrc ry = make_rsrc(a.y + n0 * T * 8, valid * row8);
    const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 32, valid * nbp * 128u);
    const Rsrc rm0 = make_rsrc(a.m0 + n0 * 32, valid * 128u);
    const Rsrc rmT = make_rsrc(a.mT + n0 * 32, valid * 128u);
    const uint32_t mo = static_cast<uint32_t>(s) * 128u + mean_off(i, j);
    const uint32_t cmo = static_cast<uint32_t>(s) * nbp * 128u + mean_off(i, j);
    v4f sq, sv0, sv1;
    auto load = [&](uint32_t t) __attribute__((always_inline)) {
      const uint32_t t0 = t * TT;
      sq = load_kq<F>(rq, row4n, s, c, t0);
      load_v<F>(sv0, sv1, rv, row8n, s, c, t0);
    };
    auto put = [&](uint32_t t) __attribute__((always_inline)) {
      float* b = in_slot(t);
      put_kq<F>(b + STile::Q, sq, c);
      put_v<F>(b + STile::V, sv0, sv1, c);
    };
    // Readouts of tile t leave its y slot as whole pieces (valid tokens only).
    auto store_y = [&](uint32_t t) __attribute__((always_inline)) {
      const float* yb = y_slot(t);
      const v4f y0 = *reinterpret_cast<const v4f*>(yb + 4 * c);
      const v4f y1 = *reinterpret_cast<const v4f*>(yb + 64 + 4 * c);
      const int len = tile_len(t);
      const uint32_t o8 = static_cast<uint32_t>(s) * row8 + static_cast<uint32_t>(t * TT) * 32u + c * 16u;
      r4::st128<r4::kNtStore>(ry, y0, (c >> 1) < len ? o8 : kOob, 0);
      r4::st128<r4::kNtStore>(ry, y1, ((c + 16) >> 1) < len ? o8 + 256u : kOob, 0);
    };
    float M0, M1;
    {
      const v2f m = own_order(r4::ld64(rm0, mo, 0), odd);
      M0 = m[0];
      M1 = m[1];
    }
    r4::vm_wait<0>();
    auto store_ckpt = [&](uint32_t rec) __attribute__((always_inline)) {
      v2f m;
      m[0] = M0;
      m[1] = M1;
      r4::st64(rbm, own_order(m, odd), cmo, rec * 128u);
    };
    store_ckpt(0);
    if (ntiles > 0) {
      load(0);
      r4::vm_wait<0>();
      put(0);
      if (ntiles > 1) load(1);
    }
    __syncthreads();
    int64_t next_ckpt = a.chunk;
    uint32_t ckpt = 1;
    for (uint32_t it = 0; it <= ntiles; ++it) {
      if (it >= 2) store_y(it - 2);
      if (it + 1 < ntiles) {
        r4::vm_wait<0>();
        put(it + 1);
        if (it + 2 < ntiles) load(it + 2);
      }
      if (it >= 1) {
        const uint32_t tl = it - 1;
        const float* b = in_slot(tl);
        const float* bu = bu_slot(tl);
        float* yb = y_slot(tl);
        const int64_t t0 = tl * TT;
        const int len = tile_len(tl);
        struct In {
          float kj, dj, qj, bu;
          v2f v;
        };
        auto read = [&](In& x, int tt) __attribute__((always_inline)) {
          x.kj = b[STile::K + 4 * tt + j];
          x.dj = FIXED ? kFixedDecay : b[STile::D + 4 * tt + j];
          x.qj = b[STile::Q + 4 * tt + j];
          x.v[0] = b[STile::V + 8 * tt + co];
          x.v[1] = b[STile::V + 8 * tt + (co ^ 1)];
          x.bu = bu[4 * tt + j];
        };
        auto ckpt_at = [&](int64_t t) __attribute__((always_inline)) {
          if (t == next_ckpt) {
            store_ckpt(ckpt++);
            next_ckpt += a.chunk;
          }
        };
        In cur, nxt;
        read(cur, 0);
        if (len == TT && a.chunk % 8 == 0) {
#pragma unroll
          for (int h = 0; h < TT / 8; ++h) {
            ckpt_at(t0 + 8 * h);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              const int tt = 8 * h + u;
              if (tt + 1 < TT) read(nxt, tt + 1);
              yb[8 * tt + co] = mean_step(M0, M1, cur.kj, cur.dj, cur.qj, cur.v, cur.bu);
              cur = nxt;
            }
          }
        } else {
          for (int tt = 0; tt < len; ++tt) {
            if (tt + 1 < len) read(nxt, tt + 1);
            ckpt_at(t0 + tt);
            yb[8 * tt + co] = mean_step(M0, M1, cur.kj, cur.dj, cur.qj, cur.v, cur.bu);
            cur = nxt;
          }
        }
      }
      __syncthreads();
    }
    if (ntiles >= 1) {
      r4::lds_wait();
      store_y(ntiles - 1);
    }
    v2f m;
    m[0] = M0;
    m[1] = M1;
    r4::st64(rmT, own_order(m, odd), mo, 0);
    store_ckpt(static_cast<uint32_t>(a.nb));
  }
}

// --------------------------------------------------- rotation dynamics forward
// The row layout for block-diagonal damped rotations (the equations of
// bssm_rotation.hip): P' = R P R^T + Q, M' = R M, u = P' k, s = r + k.u,
// beta = 1 / max(s, floor), e = v - M'^T k, M <- M' + beta u e^T,
// P <- P' - beta u u^T, y = M^T q, with R = diag of [[c, -s], [s, c]] per
// pair (c = rho cos, s = rho sin, rho = min(max(radius, tiny), 1)) and the
// pair's process variance on entry (2k, 2k).  Lane (i, j) forms
//   P'_ij = (P_ij R_ii R_jj + P_{i^1,j^1} R_{i,i^1} R_{j,j^1})
//         + (P_{i,j^1} R_ii R_{j,j^1} + P_{i^1,j} R_{i,i^1} R_jj)
// from three neighbours (quad exchange, half-row mirror + quad reversal, and
// the exchange of that); the mirror lane (j, i) forms the same products and
// sums them in the same pairs, so P stays bitwise symmetric.  The rotation
// coefficients are computed once per token and pair as the tile is staged
// (sin and cos by sincos_rad) and stored with both signs of s, so that a lane
// reads its row's (R_ii, R_{i,i^1}) as one pair; the process variances are
// stored beside zeros, which the lanes off the even diagonal read (adding a
// zero instead of selecting).  The mean pair is
// kept in the lane's own column order as in forward_kernel; its row mixing
// is one quad exchange.
struct RTile {
  // k, q [TT][4], v / y [TT][8], (c0, -s0, c0, s0, c1, -s1, c1, s1) [TT][8],
  // (p0, 0, p1, 0) [TT][4], r [TT]; sequences 8 banks apart (488 mod 32).
  static constexpr int K = 0, Q = 64, V = 128, CS = 256, PP = 384, R = 448, SEQ = 488, SIZE = SPW * SEQ;
};

template <int F = kInF32>
__global__ __launch_bounds__(kWave) void rotation_forward_kernel(RotArgs a) {
  __shared__ float tile[RTile::SIZE];
  const int lane = threadIdx.x;
  const int s = lane >> 4, c = lane & 15, i = c >> 2, j = c & 3;
  const int co = 2 * i + (j & 1);
  const bool odd = (j & 1) != 0;
  const int tr = 4 * (16 * s + 4 * j + i);  // ds_bpermute address of lane (j, i)
  // (R_ii, R_{i,i^1}) of row i: R_{i,i^1} = -s_i for an even row, +s_i for an odd one.
  const int csi_off = 4 * (i >> 1) + 2 * (i & 1), csj_off = 4 * (j >> 1) + 2 * (j & 1);
  // Process variance on the even diagonal entries only (the others read a zero).
  const int p_off = (i == j && !(i & 1)) ? 2 * (i >> 1) : 1;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t T = a.t;
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  const uint32_t row4 = static_cast<uint32_t>(T) * 16u, row8 = static_cast<uint32_t>(T) * 32u,
                 row2 = static_cast<uint32_t>(T) * 8u, row1 = static_cast<uint32_t>(T) * 4u;
  const Rsrc rk = make_rsrc(a.k + n0 * T * 4, valid * row4);
  const Rsrc rq = make_rsrc(a.q + n0 * T * 4, valid * row4);
  const Rsrc rv = make_rsrc(a.v + n0 * T * 8, valid * row8);
  const Rsrc ry = make_rsrc(a.y + n0 * T * 8, valid * row8);
  const Rsrc rrad = make_rsrc(a.rad + n0 * T * 2, valid * row2);
  const Rsrc rang = make_rsrc(a.ang + n0 * T * 2, valid * row2);
  const Rsrc rp = make_rsrc(a.p + n0 * T * 2, valid * row2);
  const Rsrc rr = make_rsrc(a.r + n0 * T, valid * row1);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 32, valid * nbp * 128u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 16, valid * nbp * 64u);
  const Rsrc rm0 = make_rsrc(a.m0 + n0 * 32, valid * 128u);
  const Rsrc rc0 = make_rsrc(a.c0 + n0 * 16, valid * 64u);
  const Rsrc rmT = make_rsrc(a.mT + n0 * 32, valid * 128u);
  const Rsrc rcT = make_rsrc(a.cT + n0 * 16, valid * 64u);
  const uint32_t mo = static_cast<uint32_t>(s) * 128u + mean_off(i, j), cvo = static_cast<uint32_t>(s) * 64u + cov_off(i, j);
  const uint32_t cmo = static_cast<uint32_t>(s) * nbp * 128u + mean_off(i, j),
                 cco = static_cast<uint32_t>(s) * nbp * 64u + cov_off(i, j);

  float P, M0, M1;
  {
    const v2f m = own_order(r4::ld64(rm0, mo, 0), odd);
    M0 = m[0];
    M1 = m[1];
    P = r4::ld32(rc0, cvo, 0);
  }
  r4::vm_wait<0>();
  auto store_ckpt = [&](uint32_t rec) __attribute__((always_inline)) {
    v2f m;
    m[0] = M0;
    m[1] = M1;
    r4::st64(rbm, own_order(m, odd), cmo, rec * 128u);
    r4::st32(rbc, P, cco, rec * 64u);
  };
  store_ckpt(0);

  // Staging: lane (s, c) moves token c's k / q piece, radii and angles (and
  // turns them into the rotation coefficients), v pieces c and c + 16, for
  // c < 8 the process piece of tokens 2c, 2c + 1, and for c < 4 the
  // observation piece of tokens 4c .. 4c + 3.
  struct RStage {
    v4f k, q, v0, v1, p, r;
    v2f rad, ang;
  };
  auto load = [&](RStage& x, uint32_t t0) __attribute__((always_inline)) {
    const uint32_t o4 = static_cast<uint32_t>(s) * row4 + (t0 + c) * 16u;
    x.k = r4::ld128<true>(rk, o4);
    x.q = r4::ld128<true>(rq, o4);
    const uint32_t o8 = static_cast<uint32_t>(s) * row8 + t0 * 32u + c * 16u;
    x.v0 = r4::ld128<true>(rv, o8);
    x.v1 = r4::ld128<true>(rv, o8 + 256u);
    const uint32_t o2 = static_cast<uint32_t>(s) * row2 + (t0 + c) * 8u;
    x.rad = r4::ld64(rrad, o2, 0);
    x.ang = r4::ld64(rang, o2, 0);
    x.p = r4::ld128<false>(rp, c < 8 ? static_cast<uint32_t>(s) * row2 + t0 * 8u + c * 16u : kOob);
    const uint32_t o1 = c < 4 ? static_cast<uint32_t>(s) * row1 + t0 * 4u + c * 16u : kOob;
    x.r = r4::ld128<false>(rr, o1);
  };
  auto put = [&](const RStage& x) __attribute__((always_inline)) {
    float* b = tile + s * RTile::SEQ;
    *reinterpret_cast<v4f*>(b + RTile::K + 4 * c) = x.k;
    *reinterpret_cast<v4f*>(b + RTile::Q + 4 * c) = x.q;
    *reinterpret_cast<v4f*>(b + RTile::V + 4 * c) = x.v0;
    *reinterpret_cast<v4f*>(b + RTile::V + 64 + 4 * c) = x.v1;
    {
      // Coefficients of token c's two pairs, as bssm_rotation.hip forms them.
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float rc = fmaxf(x.rad[e], FLT_MIN);
        const float rho = rc <= 1.f ? rc : 1.f;
        float sa, ca;
        sincos_rad(x.ang[e], sa, ca);
        const float cc = rho * ca, ss = rho * sa;
        *reinterpret_cast<v4f*>(b + RTile::CS + 8 * c + 4 * e) = v4f{cc, -ss, cc, ss};
      }
    }
    if (c < 8) {
      *reinterpret_cast<v4f*>(b + RTile::PP + 8 * c) = v4f{x.p[0], 0.f, x.p[1], 0.f};
      *reinterpret_cast<v4f*>(b + RTile::PP + 8 * c + 4) = v4f{x.p[2], 0.f, x.p[3], 0.f};
    }
    if (c < 4) *reinterpret_cast<v4f*>(b + RTile::R + 4 * c) = x.r;
  };

  struct In {
    float kj, qj, p, r;
    v2f v, csi, csj;  // (R_ii, R_{i,i^1}) and (R_jj, R_{j,j^1})
  };
  const float* mine = tile + s * RTile::SEQ;
  auto read = [&](In& x, int tt) __attribute__((always_inline)) {
    x.kj = mine[RTile::K + 4 * tt + j];
    x.qj = mine[RTile::Q + 4 * tt + j];
    x.v[0] = mine[RTile::V + 8 * tt + co];
    x.v[1] = mine[RTile::V + 8 * tt + (co ^ 1)];
    x.csi = *reinterpret_cast<const v2f*>(mine + RTile::CS + 8 * tt + csi_off);
    x.csj = *reinterpret_cast<const v2f*>(mine + RTile::CS + 8 * tt + csj_off);
    x.p = mine[RTile::PP + 4 * tt + p_off];
    x.r = mine[RTile::R + tt];
  };
  auto step = [&](const In& x) __attribute__((always_inline)) {
    const float Rii = x.csi[0], Rio = x.csi[1], Rjj = x.csj[0], Rjo = x.csj[1];
    const float x1 = dpp<kXor1>(P);         // P[i][j ^ 1]
    const float hm = dpp<kHalfMirror>(P);   // P[i ^ 1][3 - j]
    const float x2 = dpp<kQuadRev>(hm);     // P[i ^ 1][j]
    const float x3 = dpp<kXor2>(hm);        // P[i ^ 1][j ^ 1] (quad reversal, then exchange)
    const float Ps = (P * (Rii * Rjj) + x3 * (Rio * Rjo)) + (x1 * (Rii * Rjo) + x2 * (Rio * Rjj));
    const float Pp = Ps + x.p;
    const float zi = quad_sum(Pp * x.kj);  // u_i
    // u_j: u_i of the transposed lane (j, i), the bits of the column sum.
    const float zj = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(tr, __builtin_bit_cast(int, zi)));
    const float sv = quad_sum(x.kj * zj) + x.r;
    const float beta = fast_rcp(fmaxf(sv, a.floor));
    // M' = R M: row j mixes with row j ^ 1, held by lane (i, j ^ 1) in swapped order.
    const float Mp0 = fmaf(Rjj, M0, dpp<kXor1>(M1) * Rjo);
    const float Mp1 = fmaf(Rjj, M1, dpp<kXor1>(M0) * Rjo);
    const float so = own_sum(Mp0 * x.kj, Mp1 * x.kj);
    const float e0 = x.v[0] - so;
    const float e1 = x.v[1] - dpp<kXor1>(so);
    const float bu = beta * zj;
    M0 = fmaf(bu, e0, Mp0);
    M1 = fmaf(bu, e1, Mp1);
    P = fmaf(-beta, zi * zj, Pp);
    return own_sum(M0 * x.qj, M1 * x.qj);
  };

  const int64_t ntiles = (T + TT - 1) / TT;
  RStage x;
  if (ntiles > 0) load(x, 0);
  int64_t next_ckpt = a.chunk;
  uint32_t ckpt = 1;
  float* mw = tile + s * RTile::SEQ;
  v4f ys0 = v4f{0.f, 0.f, 0.f, 0.f}, ys1 = ys0;
  for (int64_t ti = 0; ti < ntiles; ++ti) {
    const uint32_t t0 = static_cast<uint32_t>(ti * TT);
    const int len = static_cast<int>((T - t0) < TT ? (T - t0) : TT);
    if (ti > 0) {
      ys0 = *reinterpret_cast<const v4f*>(mw + RTile::V + 4 * c);
      ys1 = *reinterpret_cast<const v4f*>(mw + RTile::V + 64 + 4 * c);
    }
    r4::vm_wait<0>();
    put(x);
    if (ti > 0) {
      const uint32_t o8 = static_cast<uint32_t>(s) * row8 + (t0 - TT) * 32u + c * 16u;
      r4::st128<r4::kNtStore>(ry, ys0, o8, 0);
      r4::st128<r4::kNtStore>(ry, ys1, o8 + 256u, 0);
    }
    if (ti + 1 < ntiles) load(x, t0 + TT);
    r4::lds_wait();
    if (len == TT && a.chunk % 8 == 0) {
#pragma unroll
      for (int h = 0; h < TT / 8; ++h) {
        if (static_cast<int64_t>(t0) + 8 * h == next_ckpt) {
          store_ckpt(ckpt++);
          next_ckpt += a.chunk;
        }
        In cur, nxt;
        read(cur, 8 * h);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int tt = 8 * h + u;
          if (u + 1 < 8) read(nxt, tt + 1);
          mw[RTile::V + 8 * tt + co] = step(cur);
          cur = nxt;
        }
      }
    } else {
      for (int tt = 0; tt < len; ++tt) {
        if (static_cast<int64_t>(t0) + tt == next_ckpt) {
          store_ckpt(ckpt++);
          next_ckpt += a.chunk;
        }
        In cur;
        read(cur, tt);
        mw[RTile::V + 8 * tt + co] = step(cur);
      }
    }
  }
  if (ntiles > 0) {
    const uint32_t t0 = static_cast<uint32_t>((ntiles - 1) * TT);
    const int len = static_cast<int>(T - t0);
    r4::lds_wait();
    ys0 = *reinterpret_cast<const v4f*>(mw + RTile::V + 4 * c);
    ys1 = *reinterpret_cast<const v4f*>(mw + RTile::V + 64 + 4 * c);
    const uint32_t o8 = static_cast<uint32_t>(s) * row8 + t0 * 32u + c * 16u;
    r4::st128<r4::kNtStore>(ry, ys0, (c >> 1) < len ? o8 : kOob, 0);
    r4::st128<r4::kNtStore>(ry, ys1, ((c + 16) >> 1) < len ? o8 + 256u : kOob, 0);
  }
  v2f m;
  m[0] = M0;
  m[1] = M1;
  r4::st64(rmT, own_order(m, odd), mo, 0);
  r4::st32(rcT, P, cvo, 0);
  store_ckpt(static_cast<uint32_t>(a.nb));
}

// ----------------------------------------------------------------- backward
// A 16-token tile holds two checkpoint chunks of 8 tokens (T a multiple of
// 16); tiles are visited last to first, and in each the chunk 2J + 1 before
// the chunk 2J.  A chunk is replayed from its checkpoint, keeping each
// token's belief and step intermediates in registers, and then reversed.
// Gradients overwrite their inputs in the tile (gk over k, gq over q, gd over
// d, gv over v, gp over p, gr over r) and leave with the next tile's loads.
//
// LDS per sequence: k, d, q [TT][4], v, gy [TT][8], p, r [TT]; the stride
// (mod 32 banks = 8) puts the 4 sequences' reads of one token in different
// banks.
struct BTile {
  static constexpr int K = 0, D = 64, Q = 128, V = 192, GY = 320, P = 448, R = 464, SEQ = 488, SIZE = SPW * SEQ;
};

struct BStage {
  v4f k, d, q, v0, v1, g0, g1, p, r;
};
// Gradient pieces of one tile, in the loaders' geometry.
struct GStage {
  v4f k, d, q, v0, v1, p, r;
};

struct BStreams {
  Rsrc k, d, q, v, gy, p, r;
  Rsrc gk, gd, gq, gv, gp, gr;
  uint32_t row4, row8, row1;
};

template <bool FIXED>
__device__ __forceinline__ void load_btile(BStage& x, const BStreams& st, int s, int c, uint32_t t0) {
  const uint32_t o4 = static_cast<uint32_t>(s) * st.row4 + (t0 + c) * 16u;
  x.k = r4::ld128<true>(st.k, o4);
  x.q = r4::ld128<true>(st.q, o4);
  if constexpr (!FIXED) x.d = r4::ld128<true>(st.d, o4);
  const uint32_t o8 = static_cast<uint32_t>(s) * st.row8 + t0 * 32u + c * 16u;
  x.v0 = r4::ld128<true>(st.v, o8);
  x.v1 = r4::ld128<true>(st.v, o8 + 256u);
  x.g0 = r4::ld128<true>(st.gy, o8);
  x.g1 = r4::ld128<true>(st.gy, o8 + 256u);
  if constexpr (!FIXED) {
    const uint32_t o1 = c < 4 ? static_cast<uint32_t>(s) * st.row1 + t0 * 4u + c * 16u : kOob;
    x.p = r4::ld128<false>(st.p, o1);
    x.r = r4::ld128<false>(st.r, o1);
  }
}

template <bool FIXED>
__device__ __forceinline__ void put_btile(const BStage& x, float* tl, int s, int c) {
  float* b = tl + s * BTile::SEQ;
  *reinterpret_cast<v4f*>(b + BTile::K + 4 * c) = x.k;
  *reinterpret_cast<v4f*>(b + BTile::Q + 4 * c) = x.q;
  *reinterpret_cast<v4f*>(b + BTile::V + 4 * c) = x.v0;
  *reinterpret_cast<v4f*>(b + BTile::V + 64 + 4 * c) = x.v1;
  *reinterpret_cast<v4f*>(b + BTile::GY + 4 * c) = x.g0;
  *reinterpret_cast<v4f*>(b + BTile::GY + 64 + 4 * c) = x.g1;
  if constexpr (!FIXED) {
    *reinterpret_cast<v4f*>(b + BTile::D + 4 * c) = x.d;
    if (c < 4) {
      *reinterpret_cast<v4f*>(b + BTile::P + 4 * c) = x.p;
      *reinterpret_cast<v4f*>(b + BTile::R + 4 * c) = x.r;
    }
  }
}

// The gradient pieces of a tile: read from LDS, then stored (requested
// outputs only) at the loaders' offsets.
template <bool DYN>
__device__ __forceinline__ void get_grads(GStage& g, const float* tl, int s, int c) {
  const float* b = tl + s * BTile::SEQ;
  g.k = *reinterpret_cast<const v4f*>(b + BTile::K + 4 * c);
  g.q = *reinterpret_cast<const v4f*>(b + BTile::Q + 4 * c);
  g.v0 = *reinterpret_cast<const v4f*>(b + BTile::V + 4 * c);
  g.v1 = *reinterpret_cast<const v4f*>(b + BTile::V + 64 + 4 * c);
  if constexpr (DYN) {
    g.d = *reinterpret_cast<const v4f*>(b + BTile::D + 4 * c);
    g.p = *reinterpret_cast<const v4f*>(b + BTile::P + 4 * (c & 3));
    g.r = *reinterpret_cast<const v4f*>(b + BTile::R + 4 * (c & 3));
  }
}

template <bool DYN>
__device__ __forceinline__ void store_grads(const GStage& g, const BStreams& st, const BwdArgs& a, int s, int c,
                                            uint32_t t0) {
  const uint32_t o4 = static_cast<uint32_t>(s) * st.row4 + (t0 + c) * 16u;
  r4::st128<r4::kNtStore>(st.gk, g.k, o4, 0);
  r4::st128<r4::kNtStore>(st.gq, g.q, o4, 0);
  const uint32_t o8 = static_cast<uint32_t>(s) * st.row8 + t0 * 32u + c * 16u;
  r4::st128<r4::kNtStore>(st.gv, g.v0, o8, 0);
  r4::st128<r4::kNtStore>(st.gv, g.v1, o8 + 256u, 0);
  // Without dynamics gradients, requested gd / gp / gr outputs are zero.
  const v4f zero = v4f{0.f, 0.f, 0.f, 0.f};
  if (a.gd) r4::st128<r4::kNtStore>(st.gd, DYN ? g.d : zero, o4, 0);
  const uint32_t o1 = c < 4 ? static_cast<uint32_t>(s) * st.row1 + t0 * 4u + c * 16u : kOob;
  if (a.gp) r4::st128(st.gp, DYN ? g.p : zero, o1, 0);
  if (a.gr) r4::st128(st.gr, DYN ? g.r : zero, o1, 0);
}

// Replay record of one token: the belief before it and the step's
// intermediates.
struct Hist {
  float P, M0, M1, ui, uj, s;
  v2f e;
};

// Reverse-step inputs of lane (i, j).
struct RTok {
  float ki, kj, di, dj, qj, p;
  v2f gy;  // gy[2i], gy[2i + 1]
};

template <bool FIXED>
__device__ __forceinline__ void read_rtok(RTok& x, const float* b, int tt, int i, int j) {
  x.ki = b[BTile::K + 4 * tt + i];
  x.kj = b[BTile::K + 4 * tt + j];
  x.qj = b[BTile::Q + 4 * tt + j];
  x.gy = *reinterpret_cast<const v2f*>(b + BTile::GY + 8 * tt + 2 * i);
  if constexpr (FIXED) {
    x.di = x.dj = kFixedDecay;
    x.p = kFixedProcess;
  } else {
    x.di = b[BTile::D + 4 * tt + i];
    x.dj = b[BTile::D + 4 * tt + j];
    x.p = b[BTile::P + tt];
  }
}

// The replay reads the same token inputs as the forward (v, r from the
// backward tile's regions).
template <bool FIXED>
__device__ __forceinline__ void read_ftok(Tok& x, const float* b, int tt, int i, int j) {
  x.ki = b[BTile::K + 4 * tt + i];
  x.kj = b[BTile::K + 4 * tt + j];
  x.qj = 0.f;
  x.v = *reinterpret_cast<const v2f*>(b + BTile::V + 8 * tt + 2 * i);
  if constexpr (FIXED) {
    x.di = x.dj = kFixedDecay;
    x.p = kFixedProcess;
    x.r = kFixedObservation;
  } else {
    x.di = b[BTile::D + 4 * tt + i];
    x.dj = b[BTile::D + 4 * tt + j];
    x.p = b[BTile::P + tt];
    x.r = b[BTile::R + tt];
  }
}

// x at lane (i, i) of the row, given at every lane of quad i: the transpose
// of a quantity indexed by the column j (constant down each column).
__device__ __forceinline__ float diag_pick(float x, bool i1, bool i2) {
  const float x0 = dpp<quad_perm(0, 0, 0, 0)>(x), x1 = dpp<quad_perm(1, 1, 1, 1)>(x);
  const float x2 = dpp<quad_perm(2, 2, 2, 2)>(x), x3 = dpp<quad_perm(3, 3, 3, 3)>(x);
  const float lo = i1 ? x1 : x0, hi = i1 ? x3 : x2;
  return i2 ? hi : lo;
}

// Adjoint of one token, lane (i, j).  Carried: gM0, gM1 = dL/dM[j][2i],
// dL/dM[j][2i + 1] and S = sym(dL/dP)[i][j], updated in place to their values
// before the token.  With dL/dM_new including q gy^T (the equations of
// reverse_step in bssm_rot4.h, one covariance entry per lane):
//   ge = beta gM^T u (= dL/dv),  a = gM e,  w = S u,  z = u.(a - w)
//   gs = (s > floor) ? -z beta^2 : 0 (= dL/dr),  gu = beta (a - 2 w) + gs k
//   dL/dk = -d*(M_prev ge) + gs u + P' gu  (P' = d d^T * P_prev + p I)
//   dL/dq = M_new gy,  H = S + sym(gu k^T)
//   dL/dd = 2 (H * P_prev) d + sum_c (gM - k ge^T) * M_prev,  dL/dp = trace H
//   S_prev = H * d d^T,  gM_prev = (gM - k ge^T) * d
struct ROut {
  float gk, gq, gd, gp, gs, gui, guj;
  v2f ge;
};

template <bool DYN>
__device__ __forceinline__ void reverse_step(const RTok& x, const Hist& h, float Mn0, float Mn1, float& gM0,
                                             float& gM1, float& S, float floor, float delta, bool i1, bool i2,
                                             ROut& o) {
  const float beta = fast_rcp(fmaxf(h.s, floor));
  gM0 = fmaf(x.qj, x.gy[0], gM0);
  gM1 = fmaf(x.qj, x.gy[1], gM1);
  const float ge0 = beta * quad_sum(gM0 * h.uj), ge1 = beta * quad_sum(gM1 * h.uj);
  const float a = col_sum(fmaf(gM1, h.e[1], gM0 * h.e[0]));
  const float A = col_sum(fmaf(h.M1, ge1, h.M0 * ge0));
  o.gq = col_sum(fmaf(Mn1, x.gy[1], Mn0 * x.gy[0]));
  const float gb0 = fmaf(-x.kj, ge0, gM0), gb1 = fmaf(-x.kj, ge1, gM1);
  gM0 = gb0 * x.dj;
  gM1 = gb1 * x.dj;
  const float w = col_sum(S * h.ui);  // (S u)_j
  const float z = quad_sum(h.uj * (a - w));
  const float gs = h.s > floor ? -z * beta * beta : 0.f;
  const float guj = fmaf(beta, fmaf(-2.f, w, a), gs * x.kj);
  const float gui = diag_pick(guj, i1, i2);
  const float dd = x.di * x.dj;
  const float pb = fmaf(x.p, delta, dd * h.P);
  o.gk = fmaf(-x.dj, A, gs * h.uj) + col_sum(pb * gui);
  const float H = fmaf(0.5f, gui * x.kj + guj * x.ki, S);  // bitwise symmetric with S
  if constexpr (DYN) {
    const float Bv = col_sum(fmaf(gb1, h.M1, gb0 * h.M0));
    o.gd = fmaf(2.f, col_sum((H * x.di) * h.P), Bv);
    o.gp = col_sum(quad_sum(delta * H));
  } else {
    o.gd = o.gp = 0.f;
  }
  S = H * dd;
  o.gs = gs;
  o.gui = gui;
  o.guj = guj;
  o.ge[0] = ge0;
  o.ge[1] = ge1;
}

// What the initial-covariance adjoint needs of a sequence's first token.
struct First {
  float gui, guj, ki, kj, dd;
};

template <bool FIXED, bool DYN>
__global__ __launch_bounds__(kWave) void backward_kernel(BwdArgs a) {
  __shared__ float tile[BTile::SIZE];
  const int lane = threadIdx.x;
  const int s = lane >> 4, c = lane & 15, i = c >> 2, j = c & 3;
  const float delta = i == j ? 1.f : 0.f;
  const bool i1 = (i & 1) != 0, i2 = (i & 2) != 0;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t T = a.t;
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  BStreams st;
  st.row4 = static_cast<uint32_t>(T) * 16u;
  st.row8 = static_cast<uint32_t>(T) * 32u;
  st.row1 = static_cast<uint32_t>(T) * 4u;
  st.k = make_rsrc(a.k + n0 * T * 4, valid * st.row4);
  st.q = make_rsrc(a.q + n0 * T * 4, valid * st.row4);
  st.v = make_rsrc(a.v + n0 * T * 8, valid * st.row8);
  st.gy = make_rsrc(a.gy + n0 * T * 8, valid * st.row8);
  st.d = make_rsrc(FIXED ? a.k : a.d + n0 * T * 4, FIXED ? 0u : valid * st.row4);
  st.p = make_rsrc(FIXED ? a.k : a.p + n0 * T, FIXED ? 0u : valid * st.row1);
  st.r = make_rsrc(FIXED ? a.k : a.r + n0 * T, FIXED ? 0u : valid * st.row1);
  st.gk = make_rsrc(a.gk + n0 * T * 4, valid * st.row4);
  st.gq = make_rsrc(a.gq + n0 * T * 4, valid * st.row4);
  st.gv = make_rsrc(a.gv + n0 * T * 8, valid * st.row8);
  st.gd = make_rsrc(a.gd ? a.gd + n0 * T * 4 : a.gk, a.gd ? valid * st.row4 : 0u);
  st.gp = make_rsrc(a.gp ? a.gp + n0 * T : a.gk, a.gp ? valid * st.row1 : 0u);
  st.gr = make_rsrc(a.gr ? a.gr + n0 * T : a.gk, a.gr ? valid * st.row1 : 0u);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 32, valid * nbp * 128u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 16, valid * nbp * 64u);
  const uint32_t mo = static_cast<uint32_t>(s) * 128u + mean_off(i, j), co = static_cast<uint32_t>(s) * 64u + cov_off(i, j);
  const uint32_t cmo = static_cast<uint32_t>(s) * nbp * 128u + mean_off(i, j),
                 cco = static_cast<uint32_t>(s) * nbp * 64u + cov_off(i, j);

  // Carried adjoints from the final-state gradients (null: zero).
  float gM0, gM1, S;
  {
    const bool has_m = a.gmf != nullptr, has_c = a.gcf != nullptr;
    const Rsrc rgm = make_rsrc(has_m ? a.gmf + n0 * 32 : a.k, has_m ? valid * 128u : 0u);
    const Rsrc rgc = make_rsrc(has_c ? a.gcf + n0 * 16 : a.k, has_c ? valid * 64u : 0u);
    const v2f m = r4::ld64(rgm, mo, 0);
    gM0 = m[0];
    gM1 = m[1];
    const uint32_t tr = static_cast<uint32_t>(s) * 64u + cov_off(j, i);
    S = 0.5f * (r4::ld32(rgc, co, 0) + r4::ld32(rgc, tr, 0));
  }
  auto load_ckpt = [&](Bel& b, int64_t rec) __attribute__((always_inline)) {
    const v2f m = r4::ld64(rbm, cmo + static_cast<uint32_t>(rec) * 128u, 0);
    b.M0 = m[0];
    b.M1 = m[1];
    b.P = r4::ld32(rbc, cco + static_cast<uint32_t>(rec) * 64u, 0);
  };

  float* mine = tile + s * BTile::SEQ;
  First first = {0.f, 0.f, 0.f, 0.f, 0.f};
  // Replay and reverse of the chunk at tile token base (0 or 8).
  auto run_chunk = [&](Bel b, int base) __attribute__((always_inline)) {
    Hist h[8];
    {
      Tok cur, nxt;
      read_ftok<FIXED>(cur, mine, base, i, j);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (u + 1 < 8) read_ftok<FIXED>(nxt, mine, base + u + 1, i, j);
        h[u].P = b.P;
        h[u].M0 = b.M0;
        h[u].M1 = b.M1;
        StepOut o;
        forward_step<false>(b, cur, delta, a.floor, o);
        h[u].ui = o.ui;
        h[u].uj = o.uj;
        h[u].s = o.s;
        h[u].e = o.e;
        cur = nxt;
      }
    }
    RTok cur, nxt;
    read_rtok<FIXED>(cur, mine, base + 7, i, j);
#pragma unroll
    for (int u = 7; u >= 0; --u) {
      const int tt = base + u;
      if (u > 0) read_rtok<FIXED>(nxt, mine, tt - 1, i, j);
      // The mean after the token: the next token's record, or the replayed
      // belief after the chunk's last token.
      const float Mn0 = u < 7 ? h[u < 7 ? u + 1 : u].M0 : b.M0;
      const float Mn1 = u < 7 ? h[u < 7 ? u + 1 : u].M1 : b.M1;
      ROut o;
      reverse_step<DYN>(cur, h[u], Mn0, Mn1, gM0, gM1, S, a.floor, delta, i1, i2, o);
      mine[BTile::K + 4 * tt + j] = o.gk;
      mine[BTile::Q + 4 * tt + j] = o.gq;
      mine[BTile::V + 8 * tt + 2 * i + (j & 1)] = (j & 1) ? o.ge[1] : o.ge[0];
      if constexpr (DYN) {
        mine[BTile::D + 4 * tt + j] = o.gd;
        mine[BTile::P + tt] = o.gp;
        mine[BTile::R + tt] = o.gs;
      }
      if (u == 0) {
        first.gui = o.gui;
        first.guj = o.guj;
        first.ki = cur.ki;
        first.kj = cur.kj;
        first.dd = cur.di * cur.dj;
      }
      cur = nxt;
    }
  };

  const int64_t ntiles = T / TT;
  BStage x;
  Bel nk0, nk1;
  if (ntiles > 0) {
    load_btile<FIXED>(x, st, s, c, static_cast<uint32_t>((ntiles - 1) * TT));
    load_ckpt(nk0, 2 * (ntiles - 1));
    load_ckpt(nk1, 2 * (ntiles - 1) + 1);
  }
  GStage go;
  for (int64_t ti = ntiles - 1; ti >= 0; --ti) {
    const uint32_t t0 = static_cast<uint32_t>(ti * TT);
    // The next tile's gradients leave LDS before this tile lands there.
    if (ti + 1 < ntiles) get_grads<DYN>(go, tile, s, c);
    r4::vm_wait<0>();
    const Bel k0 = nk0, k1 = nk1;
    put_btile<FIXED>(x, tile, s, c);
    if (ti + 1 < ntiles) store_grads<DYN>(go, st, a, s, c, t0 + TT);
    if (ti > 0) {
      load_btile<FIXED>(x, st, s, c, t0 - TT);
      load_ckpt(nk0, 2 * ti - 2);
      load_ckpt(nk1, 2 * ti - 1);
    }
    r4::lds_wait();
    run_chunk(k1, 8);
    run_chunk(k0, 0);
  }
  if (ntiles > 0) {
    r4::lds_wait();
    get_grads<DYN>(go, tile, s, c);
    store_grads<DYN>(go, st, a, s, c, 0);
  }
  if (a.gm0) {
    const Rsrc rgm0 = make_rsrc(a.gm0 + n0 * 32, valid * 128u);
    v2f m;
    m[0] = gM0;
    m[1] = gM1;
    r4::st64(rgm0, m, mo, 0);
  }
  if (a.gc0) {
    // The full (asymmetric) derivative for the covariance entering the first
    // token: S + (gu k^T - sym(gu k^T)) * d d^T.
    const Rsrc rgc0 = make_rsrc(a.gc0 + n0 * 16, valid * 64u);
    const float asym = 0.5f * (first.gui * first.kj - first.guj * first.ki);
    r4::st32(rgc0, fmaf(asym, first.dd, S), co, 0);
  }
}

// ---------------------------------------------- three-wave backward (split)
// A wave issues at most one instruction every ~6 cycles, so at the smallest
// batches (one wave per SIMD or fewer) each wave's time is its instruction
// count.  The backward splits three ways: the mean adjoint (gM, ge = dL/dv,
// dL/dq) needs of the covariance side only u and beta; the covariance
// adjoint (S, gu, dL/dk, dL/dd, dL/dp, dL/dr) needs of the mean side only
// three column sums per token, a = gM e, A = M_prev ge and sum_c gb M_prev;
// and the covariance replay feeds both.  A workgroup of three waves holds the
// same 4 sequences and walks the checkpoint chunks (8 tokens) last to first
// in steps, one barrier per step.  With x the chunk's position in that
// order, at step x:
//   wave 0 replays the covariance of chunk x (its records P, u, s go to
//          LDS, and u_j and beta for the mean wave);
//   wave 2 replays and reverses the mean of chunk x - 1 (from u and beta)
//          and leaves the three sums;
//   wave 1 reverses the covariance of chunk x - 2 (from the records and the
//          sums).
// Wave 0 also moves every stream of the loop: it stages k, d, p, r, q, v, gy
// and both checkpoints one step ahead and stores the gradients (gq, gv one
// step after wave 2 leaves them, gk, gd, gp, gr one step after wave 1), so
// the two long waves never wait for global memory (a wait for loads is also a
// wait for the stores issued with them).  The operations are those of
// backward_kernel in its order: the results are bitwise the same.
struct SBTile {
  static constexpr int CH = 8;
  // Chunk slot per sequence (5 slots: a chunk is staged one step before its
  // replay and its last gradients leave three steps after): k, d, q [CH][4],
  // v, gy [CH][8], p, r [CH], and the mean checkpoint (2 per lane).
  static constexpr int K = 0, D = 32, Q = 64, V = 96, GY = 160, P = 224, R = 232, MC = 264, SEQ = 296,
                       SLOT = SPW * SEQ;
  static constexpr int NSLOT = 5;
  // Covariance to mean (2 slots): u_j [CH][4], beta [CH].
  static constexpr int USEQ = 40, USLOT = SPW * USEQ;
  // Mean to covariance (2 slots): a, A, sum_c gb M_prev [CH][4] each.
  static constexpr int ASEQ = 104, ASLOT = SPW * ASEQ;
  // Covariance records (3 slots: written at step x, read at step x + 2):
  // [CH][64 lanes] of (P, u_i, u_j, s).
  static constexpr int RSLOT = CH * kWave * 4;
  static constexpr int IN = 0, U = NSLOT * SLOT, A = U + 2 * USLOT, REC = A + 2 * ASLOT, SIZE = REC + 3 * RSLOT;
};

// Covariance record of one replayed token (one 16-byte LDS word per lane).
struct PRec {
  float P, ui, uj, s;
};
__device__ __forceinline__ v4f pack(const PRec& r) { return v4f{r.P, r.ui, r.uj, r.s}; }
__device__ __forceinline__ PRec unpack(v4f x) { return PRec{x[0], x[1], x[2], x[3]}; }
// Mean record of one replayed token (record order, as backward_kernel).
struct MRec {
  float M0, M1;
  v2f e;
};

// Mean half of the reverse (reverse_step's gM, ge, a, A, C, gb, Bv).
template <bool DYN>
__device__ __forceinline__ void mean_reverse(float kj, float dj, float qj, v2f gy, const MRec& h, float uj, float beta,
                                             float Mn0, float Mn1, float& gM0, float& gM1, float& a_out,
                                             float& A_out, float& Bv_out, float& gq, float& ge0, float& ge1) {
  gM0 = fmaf(qj, gy[0], gM0);
  gM1 = fmaf(qj, gy[1], gM1);
  ge0 = beta * quad_sum(gM0 * uj);
  ge1 = beta * quad_sum(gM1 * uj);
  a_out = col_sum(fmaf(gM1, h.e[1], gM0 * h.e[0]));
  A_out = col_sum(fmaf(h.M1, ge1, h.M0 * ge0));
  gq = col_sum(fmaf(Mn1, gy[1], Mn0 * gy[0]));
  const float gb0 = fmaf(-kj, ge0, gM0), gb1 = fmaf(-kj, ge1, gM1);
  gM0 = gb0 * dj;
  gM1 = gb1 * dj;
  Bv_out = DYN ? col_sum(fmaf(gb1, h.M1, gb0 * h.M0)) : 0.f;
}

// Covariance half of the reverse (reverse_step's w, z, gs, gu, gk, H, gd,
// gp, S).
template <bool DYN>
__device__ __forceinline__ void cov_reverse(float ki, float kj, float di, float dj, float p, const PRec& h, float a,
                                            float A, float Bv, float& S, float floor, float delta, bool i1, bool i2,
                                            ROut& o) {
  const float beta = fast_rcp(fmaxf(h.s, floor));
  const float w = col_sum(S * h.ui);
  const float z = quad_sum(h.uj * (a - w));
  const float gs = h.s > floor ? -z * beta * beta : 0.f;
  const float guj = fmaf(beta, fmaf(-2.f, w, a), gs * kj);
  const float gui = diag_pick(guj, i1, i2);
  const float dd = di * dj;
  const float pb = fmaf(p, delta, dd * h.P);
  o.gk = fmaf(-dj, A, gs * h.uj) + col_sum(pb * gui);
  const float H = fmaf(0.5f, gui * kj + guj * ki, S);
  if constexpr (DYN) {
    o.gd = fmaf(2.f, col_sum((H * di) * h.P), Bv);
    o.gp = col_sum(quad_sum(delta * H));
  } else {
    o.gd = o.gp = 0.f;
  }
  S = H * dd;
  o.gs = gs;
  o.gui = gui;
  o.guj = guj;
}

// G groups of SPW sequences per workgroup, three waves each, one barrier for
// all.  A workgroup's waves go to the CU's SIMDs in the cyclic order 0, 2, 1,
// 3 (an HW_ID probe on MI355X), and two workgroups on one CU start at varying
// points of it, so with two three-wave workgroups per CU two long waves can
// share a SIMD.  With G = 2 the six waves are ordered reverse A, reverse B,
// mean A, mean B, replay A, replay B: waves 4 and 5 share the SIMDs of waves 0
// and 1, and every long wave has its SIMD alone or with a replay wave.
template <bool FIXED, bool DYN, int F, int G>
__global__ __launch_bounds__(3 * G * kWave) void backward_split_kernel(BwdArgs a) {
  __shared__ float lds_all[G * SBTile::SIZE];
  constexpr int CH = SBTile::CH;
  // The wave index, uniform across the wave (so are role, group and their
  // addresses and buffer descriptors).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // role 0: covariance replay and the streams, 1: covariance reverse, 2: mean.
  const int role = G == 1 ? wave : (wave < 2 ? 1 : wave < 4 ? 2 : 0);
  const int grp = G == 1 ? 0 : (wave & 1);
  float* const lds = lds_all + grp * SBTile::SIZE;
  const int s = lane >> 4, c = lane & 15, i = c >> 2, j = c & 3;
  const float delta = i == j ? 1.f : 0.f;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * G + grp) * SPW;
  const int64_t T = a.t;
  const int64_t rest = a.n - n0;  // the last workgroup's second group may hold none
  const uint32_t valid = static_cast<uint32_t>(rest <= 0 ? 0 : rest < SPW ? rest : SPW);
  const uint32_t row4 = static_cast<uint32_t>(T) * 16u, row8 = static_cast<uint32_t>(T) * 32u,
                 row1 = static_cast<uint32_t>(T) * 4u;
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const int64_t nb = T / CH;  // chunks; position x is chunk nb - 1 - x
  // Ring slots of step position x (T / 8 positions: 32-bit arithmetic).
  auto slot = [&](int64_t x) __attribute__((always_inline)) {
    return lds + SBTile::IN + static_cast<int>(static_cast<uint32_t>(x) % SBTile::NSLOT) * SBTile::SLOT +
           s * SBTile::SEQ;
  };
  auto uslot = [&](int64_t x) __attribute__((always_inline)) {
    return lds + SBTile::U + static_cast<int>(x & 1) * SBTile::USLOT + s * SBTile::USEQ;
  };
  auto aslot = [&](int64_t x) __attribute__((always_inline)) {
    return lds + SBTile::A + static_cast<int>(x & 1) * SBTile::ASLOT + s * SBTile::ASEQ;
  };
  auto rslot = [&](int64_t x) __attribute__((always_inline)) {
    return lds + SBTile::REC + static_cast<int>(static_cast<uint32_t>(x) % 3u) * SBTile::RSLOT + 4 * lane;
  };
  // First token of chunk position x.
  auto tok0 = [&](int64_t x) __attribute__((always_inline)) { return static_cast<uint32_t>((nb - 1 - x) * CH); };
  const uint32_t o4 = static_cast<uint32_t>(s) * row4 + static_cast<uint32_t>(c) * 16u;  // + t0 * 16
  const uint32_t o8 = static_cast<uint32_t>(s) * row8 + static_cast<uint32_t>(c) * 16u;  // + t0 * 32
  const uint32_t o1 = static_cast<uint32_t>(s) * row1 + static_cast<uint32_t>(c) * 16u;  // + t0 * 4
  // Bytes per sequence row of k, q (and gk, gq) and of v (and gv) in format F.
  const uint32_t row4n = static_cast<uint32_t>(T) * kq_bytes<F>(), row8n = 2u * row4n;

  if (role == 0) {
    // ------------------------------------------------ covariance replay wave
    const Rsrc rk = make_rsrc(r4::byte_offset(a.k, n0 * row4n), valid * row4n);
    const Rsrc rd = make_rsrc(FIXED ? a.k : a.d + n0 * T * 4, FIXED ? 0u : valid * row4);
    const Rsrc rp = make_rsrc(FIXED ? a.k : a.p + n0 * T, FIXED ? 0u : valid * row1);
    const Rsrc rr = make_rsrc(FIXED ? a.k : a.r + n0 * T, FIXED ? 0u : valid * row1);
    const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 16, valid * nbp * 64u);
    const Rsrc rq = make_rsrc(r4::byte_offset(a.q, n0 * row4n), valid * row4n);
    const Rsrc rv = make_rsrc(r4::byte_offset(a.v, n0 * row8n), valid * row8n);
    const Rsrc rgy = make_rsrc(a.gy + n0 * T * 8, valid * row8);
    const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 32, valid * nbp * 128u);
    const uint32_t cco = static_cast<uint32_t>(s) * nbp * 64u + cov_off(i, j);
    const uint32_t cmo = static_cast<uint32_t>(s) * nbp * 128u + mean_off(i, j);
    v4f sk, sd, sp, sr, sq, sv, sv1, sg;
    v2f sm;
    auto load = [&](int64_t x) __attribute__((always_inline)) {
      const uint32_t t0 = tok0(x);
      const uint32_t q4 = c < CH ? o4 + t0 * 16u : kOob;
      sk = load_kq<F, CH>(rk, row4n, s, c, t0);
      if constexpr (!FIXED) {
        sd = r4::ld128<true>(rd, q4);
        const uint32_t q1 = c < CH / 4 ? o1 + t0 * 4u : kOob;
        sp = r4::ld128<false>(rp, q1);
        sr = r4::ld128<false>(rr, q1);
      }
      sq = load_kq<F, CH>(rq, row4n, s, c, t0);
      load_v<F, CH>(sv, sv1, rv, row8n, s, c, t0);
      sg = r4::ld128<true>(rgy, o8 + t0 * 32u);
      sm = r4::ld64(rbm, cmo + static_cast<uint32_t>(nb - 1 - x) * 128u, 0);
    };
    auto put = [&](int64_t x) __attribute__((always_inline)) {
      float* b = slot(x);
      put_kq<F, CH>(b + SBTile::K, sk, c);
      if constexpr (!FIXED) {
        if (c < CH) *reinterpret_cast<v4f*>(b + SBTile::D + 4 * c) = sd;
      }
      if constexpr (!FIXED) {
        if (c < CH / 4) {
          *reinterpret_cast<v4f*>(b + SBTile::P + 4 * c) = sp;
          *reinterpret_cast<v4f*>(b + SBTile::R + 4 * c) = sr;
        }
      }
      put_kq<F, CH>(b + SBTile::Q, sq, c);
      put_v<F, CH>(b + SBTile::V, sv, sv1, c);
      *reinterpret_cast<v4f*>(b + SBTile::GY + 4 * c) = sg;
      *reinterpret_cast<v2f*>(b + SBTile::MC + 2 * c) = sm;
    };
    auto ckpt = [&](int64_t x) __attribute__((always_inline)) {
      return r4::ld32(rbc, cco + static_cast<uint32_t>(nb - 1 - x) * 64u, 0);
    };
    // Gradients of chunk position x leave its slot (requested outputs; zero
    // gd / gp / gr without dynamics gradients): gq, gv from the mean wave,
    // gk, gd, gp, gr from the covariance reverse wave.
    const Rsrc rgq = make_rsrc(r4::byte_offset(a.gq, n0 * row4n), valid * row4n);
    const Rsrc rgv = make_rsrc(r4::byte_offset(a.gv, n0 * row8n), valid * row8n);
    const Rsrc rgk = make_rsrc(r4::byte_offset(a.gk, n0 * row4n), valid * row4n);
    const Rsrc rgd = make_rsrc(a.gd ? a.gd + n0 * T * 4 : a.gk, a.gd ? valid * row4 : 0u);
    const Rsrc rgp = make_rsrc(a.gp ? a.gp + n0 * T : a.gk, a.gp ? valid * row1 : 0u);
    const Rsrc rgr = make_rsrc(a.gr ? a.gr + n0 * T : a.gk, a.gr ? valid * row1 : 0u);
    auto store_mean = [&](int64_t x) __attribute__((always_inline)) {
      const float* b = slot(x);
      const uint32_t t0 = tok0(x);
      store_kq<F, CH>(rgq, row4n, s, c, t0, b + SBTile::Q);
      store_v<F, CH>(rgv, row8n, s, c, t0, b + SBTile::V);
    };
    auto store_cov = [&](int64_t x) __attribute__((always_inline)) {
      const float* b = slot(x);
      const uint32_t t0 = tok0(x);
      const uint32_t q4 = c < CH ? o4 + t0 * 16u : kOob, q1 = c < CH / 4 ? o1 + t0 * 4u : kOob;
      const v4f zero = v4f{0.f, 0.f, 0.f, 0.f};
      const int c8 = c & (CH - 1), c2 = c & (CH / 4 - 1);
      store_kq<F, CH>(rgk, row4n, s, c, t0, b + SBTile::K);
      if (a.gd) r4::st128<r4::kNtStore>(rgd, DYN ? *reinterpret_cast<const v4f*>(b + SBTile::D + 4 * c8) : zero, q4, 0);
      if (a.gp) r4::st128(rgp, DYN ? *reinterpret_cast<const v4f*>(b + SBTile::P + 4 * c2) : zero, q1, 0);
      if (a.gr) r4::st128(rgr, DYN ? *reinterpret_cast<const v4f*>(b + SBTile::R + 4 * c2) : zero, q1, 0);
    };
    float Pload = 0.f;
    if (nb > 0) {
      load(0);
      Pload = ckpt(0);
      r4::vm_wait<0>();
      put(0);
      if (nb > 1) load(1);
    }
    __syncthreads();
    struct In {
      float ki, kj, di, dj, p, r;
    };
    for (int64_t x = 0; x <= nb + 1; ++x) {
      r4::vm_wait<0>();
      float Pc = Pload;
      if (x + 1 < nb) {
        Pload = ckpt(x + 1);
        put(x + 1);
        if (x + 2 < nb) load(x + 2);
      }
      if (x >= 2) store_mean(x - 2);
      if (x >= 3) store_cov(x - 3);
      if (x < nb) {
        const float* pb = slot(x);
        float* ub = uslot(x);
        float* rec = rslot(x);
        auto read = [&](In& y, int k) __attribute__((always_inline)) {
          y.ki = pb[SBTile::K + 4 * k + i];
          y.kj = pb[SBTile::K + 4 * k + j];
          y.di = FIXED ? kFixedDecay : pb[SBTile::D + 4 * k + i];
          y.dj = FIXED ? kFixedDecay : pb[SBTile::D + 4 * k + j];
          y.p = FIXED ? kFixedProcess : pb[SBTile::P + k];
          y.r = FIXED ? kFixedObservation : pb[SBTile::R + k];
        };
        In cur, nxt;
        read(cur, 0);
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          if (k + 1 < CH) read(nxt, k + 1);
          // forward_step's covariance operations, in its order.
          PRec h;
          h.P = Pc;
          const float wki = cur.di * cur.ki, wkj = cur.dj * cur.kj;
          const float zi = quad_sum(Pc * wkj);
          const float zj = col_sum(Pc * wki);
          const float ui = fmaf(cur.di, zi, cur.p * cur.ki), uj = fmaf(cur.dj, zj, cur.p * cur.kj);
          const float sv = quad_sum(cur.kj * uj) + cur.r;
          const float beta = fast_rcp(fmaxf(sv, a.floor));
          const float dp = fmaf(cur.p, delta, (cur.di * cur.dj) * Pc);
          Pc = fmaf(-beta, ui * uj, dp);
          h.ui = ui;
          h.uj = uj;
          h.s = sv;
          *reinterpret_cast<v4f*>(rec + k * 4 * kWave) = pack(h);
          ub[4 * k + j] = uj;
          ub[4 * CH + k] = beta;
          cur = nxt;
        }
      }
      __syncthreads();
    }
    if (nb > 0) store_cov(nb - 1);
  } else if (role == 1) {
    // ------------------------------------------------ covariance reverse wave
    const bool i1 = (i & 1) != 0, i2 = (i & 2) != 0;
    const uint32_t cvo = static_cast<uint32_t>(s) * 64u + cov_off(i, j);
    float S;
    {
      const bool has_c = a.gcf != nullptr;
      const Rsrc rgc = make_rsrc(has_c ? a.gcf + n0 * 16 : a.k, has_c ? valid * 64u : 0u);
      const uint32_t tr = static_cast<uint32_t>(s) * 64u + cov_off(j, i);
      S = 0.5f * (r4::ld32(rgc, cvo, 0) + r4::ld32(rgc, tr, 0));
    }
    First first = {0.f, 0.f, 0.f, 0.f, 0.f};
    __syncthreads();
    struct In {
      float ki, kj, di, dj, p, a, A, Bv;
      v4f rec;
    };
    for (int64_t x = 0; x <= nb + 1; ++x) {
      if (x >= 2) {
        float* rb = slot(x - 2);
        const float* ab = aslot(x - 2);
        const float* rec = rslot(x - 2);
        auto read = [&](In& y, int u) __attribute__((always_inline)) {
          y.ki = rb[SBTile::K + 4 * u + i];
          y.kj = rb[SBTile::K + 4 * u + j];
          y.di = FIXED ? kFixedDecay : rb[SBTile::D + 4 * u + i];
          y.dj = FIXED ? kFixedDecay : rb[SBTile::D + 4 * u + j];
          y.p = FIXED ? kFixedProcess : rb[SBTile::P + u];
          y.a = ab[4 * u + j];
          y.A = ab[4 * CH + 4 * u + j];
          y.Bv = DYN ? ab[8 * CH + 4 * u + j] : 0.f;
          y.rec = *reinterpret_cast<const v4f*>(rec + u * 4 * kWave);
        };
        In cur, nxt;
        read(cur, CH - 1);
#pragma unroll
        for (int u = CH - 1; u >= 0; --u) {
          if (u > 0) read(nxt, u - 1);
          ROut o;
          cov_reverse<DYN>(cur.ki, cur.kj, cur.di, cur.dj, cur.p, unpack(cur.rec), cur.a, cur.A, cur.Bv, S, a.floor,
                           delta, i1, i2, o);
          rb[SBTile::K + 4 * u + j] = o.gk;
          if constexpr (DYN) {
            rb[SBTile::D + 4 * u + j] = o.gd;
            rb[SBTile::P + u] = o.gp;
            rb[SBTile::R + u] = o.gs;
          }
          if (u == 0) {
            first.gui = o.gui;
            first.guj = o.guj;
            first.ki = cur.ki;
            first.kj = cur.kj;
            first.dd = cur.di * cur.dj;
          }
          cur = nxt;
        }
      }
      __syncthreads();
    }
    if (a.gc0) {
      const Rsrc rgc0 = make_rsrc(a.gc0 + n0 * 16, valid * 64u);
      const float asym = 0.5f * (first.gui * first.kj - first.guj * first.ki);
      r4::st32(rgc0, fmaf(asym, first.dd, S), cvo, 0);
    }
  } else {
    // ------------------------------------------------ mean wave
    const uint32_t mo = static_cast<uint32_t>(s) * 128u + mean_off(i, j);
    float gM0, gM1;
    {
      const bool has_m = a.gmf != nullptr;
      const Rsrc rgm = make_rsrc(has_m ? a.gmf + n0 * 32 : a.k, has_m ? valid * 128u : 0u);
      const v2f m = r4::ld64(rgm, mo, 0);
      gM0 = m[0];
      gM1 = m[1];
    }
    __syncthreads();
    for (int64_t x = 0; x <= nb + 1; ++x) {
      if (x >= 1 && x <= nb) {
        float* b = slot(x - 1);
        const float* ub = uslot(x - 1);
        float* ab = aslot(x - 1);
        MRec h[CH];
        const v2f Mc = *reinterpret_cast<const v2f*>(b + SBTile::MC + 2 * c);  // checkpoint of the chunk
        float M0 = Mc[0], M1 = Mc[1];
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          const float kj = b[SBTile::K + 4 * k + j];
          const float dj = FIXED ? kFixedDecay : b[SBTile::D + 4 * k + j];
          const v2f v = *reinterpret_cast<const v2f*>(b + SBTile::V + 8 * k + 2 * i);
          const float uj = ub[4 * k + j], beta = ub[4 * CH + k];
          // forward_step's mean operations, in its order.
          h[k].M0 = M0;
          h[k].M1 = M1;
          const float wkj = dj * kj;
          const float e0 = v[0] - quad_sum(M0 * wkj);
          const float e1 = v[1] - quad_sum(M1 * wkj);
          const float bu = beta * uj;
          M0 = fmaf(bu, e0, dj * M0);
          M1 = fmaf(bu, e1, dj * M1);
          h[k].e[0] = e0;
          h[k].e[1] = e1;
        }
        struct In {
          float kj, dj, qj, uj, beta;
          v2f gy;
        };
        auto read = [&](In& y, int u) __attribute__((always_inline)) {
          y.kj = b[SBTile::K + 4 * u + j];
          y.dj = FIXED ? kFixedDecay : b[SBTile::D + 4 * u + j];
          y.qj = b[SBTile::Q + 4 * u + j];
          y.gy = *reinterpret_cast<const v2f*>(b + SBTile::GY + 8 * u + 2 * i);
          y.uj = ub[4 * u + j];
          y.beta = ub[4 * CH + u];
        };
        In cur, nxt;
        read(cur, CH - 1);
#pragma unroll
        for (int u = CH - 1; u >= 0; --u) {
          if (u > 0) read(nxt, u - 1);
          const float Mn0 = u < CH - 1 ? h[u < CH - 1 ? u + 1 : u].M0 : M0;
          const float Mn1 = u < CH - 1 ? h[u < CH - 1 ? u + 1 : u].M1 : M1;
          float av, Av, Bv, gq, ge0, ge1;
          mean_reverse<DYN>(cur.kj, cur.dj, cur.qj, cur.gy, h[u], cur.uj, cur.beta, Mn0, Mn1, gM0, gM1, av, Av, Bv,
                            gq, ge0, ge1);
          ab[4 * u + j] = av;
          ab[4 * CH + 4 * u + j] = Av;
          if constexpr (DYN) ab[8 * CH + 4 * u + j] = Bv;
          b[SBTile::Q + 4 * u + j] = gq;
          b[SBTile::V + 8 * u + 2 * i + (j & 1)] = (j & 1) ? ge1 : ge0;
          cur = nxt;
        }
      }
      __syncthreads();
    }
    if (a.gm0) {
      const Rsrc rgm0 = make_rsrc(a.gm0 + n0 * 32, valid * 128u);
      v2f m;
      m[0] = gM0;
      m[1] = gM1;
      r4::st64(rgm0, m, mo, 0);
    }
  }
}

}  // namespace
}  // namespace sn

namespace {
// Measured crossovers against the rotated-layout kernels (T = 512): the row
// forward is faster up to about 24576 sequences and level beyond, the row
// backward up to about 8192; the two-wave forward beats the one-wave row
// forward up to 2048 (by 15 % at 1024 and below, 4 % at 2048), the
// three-wave backward the one-wave one up to 2048 (30 %, 12 %; beyond that
// its 50 KB of LDS per workgroup leave too few workgroups per CU).
std::atomic<int64_t> g_small_limit[5] = {{24576}, {8192}, {2048}, {2048}, {32768}};
}  // namespace

int64_t small_batch_limit(int direction) { return g_small_limit[direction].load(std::memory_order_relaxed); }
int64_t set_small_batch_limit(int direction, int64_t limit) {
  return g_small_limit[direction].exchange(limit, std::memory_order_relaxed);
}

namespace {
// Sequences up to which one group per workgroup leaves a CU to every
// workgroup (4 sequences each, 256 CUs); the split kernels put two groups in
// a workgroup beyond it.
constexpr int64_t kSplitGroupsAbove = 4 * 256;

// bf16 / float8 streams run the two-wave kernel only (the dispatch keeps them
// within its limit).
template <int F, int G>
void launch_forward_split(bool fixed, const FwdArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((a.n + G * sn::SPW - 1) / (G * sn::SPW))), block(2 * G * kWave);
  if (fixed) hipLaunchKernelGGL((sn::forward_split_kernel<true, F, G>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((sn::forward_split_kernel<false, F, G>), grid, block, 0, stream, a);
}

template <int F>
hipError_t launch_forward_small_fmt(bool fixed, const FwdArgs& a, int64_t blocks, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(blocks));
  if (F != kInF32 || a.n <= small_batch_limit(2)) {
    // One group per workgroup while every workgroup has a CU of its own.
    if (a.n > kSplitGroupsAbove) launch_forward_split<F, 2>(fixed, a, stream);
    else launch_forward_split<F, 1>(fixed, a, stream);
  } else if constexpr (F == kInF32) {
    if (fixed) hipLaunchKernelGGL((sn::forward_kernel<true, F>), grid, dim3(kWave), 0, stream, a);
    else hipLaunchKernelGGL((sn::forward_kernel<false, F>), grid, dim3(kWave), 0, stream, a);
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_forward_small(bool fixed, const FwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + sn::SPW - 1) / sn::SPW;
  if (blocks == 0) return hipSuccess;
  switch (a.in_fmt) {
    case kInBf16: return launch_forward_small_fmt<kInBf16>(fixed, a, blocks, stream);
    case kInE4M3: return launch_forward_small_fmt<kInE4M3>(fixed, a, blocks, stream);
    case kInE5M2: return launch_forward_small_fmt<kInE5M2>(fixed, a, blocks, stream);
    default: return launch_forward_small_fmt<kInF32>(fixed, a, blocks, stream);
  }
}

namespace {
template <int F, int G>
void launch_backward_split_g(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((a.n + G * sn::SPW - 1) / (G * sn::SPW))), block(3 * G * kWave);
  if (fixed) hipLaunchKernelGGL((sn::backward_split_kernel<true, false, F, G>), grid, block, 0, stream, a);
  else if (dyn) hipLaunchKernelGGL((sn::backward_split_kernel<false, true, F, G>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((sn::backward_split_kernel<false, false, F, G>), grid, block, 0, stream, a);
}
// One group per workgroup while every workgroup has a CU of its own; beyond
// that two groups per workgroup (one workgroup per CU up to 2048 sequences).
template <int F>
void launch_backward_split(bool fixed, bool dyn, const BwdArgs& a, dim3, hipStream_t stream) {
  if (a.n > static_cast<int64_t>(kSplitGroupsAbove)) launch_backward_split_g<F, 2>(fixed, dyn, a, stream);
  else launch_backward_split_g<F, 1>(fixed, dyn, a, stream);
}
}  // namespace

// bf16 / float8 streams run the three-wave kernel only (the dispatch keeps
// them within its limit).
hipError_t launch_backward_small(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  if (a.t % sn::TT != 0 || a.chunk != kRot4Chunk) return hipErrorInvalidValue;
  const int64_t blocks = (a.n + sn::SPW - 1) / sn::SPW;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks));
  switch (a.in_fmt) {
    case kInBf16: launch_backward_split<kInBf16>(fixed, dyn, a, grid, stream); return hipGetLastError();
    case kInE4M3: launch_backward_split<kInE4M3>(fixed, dyn, a, grid, stream); return hipGetLastError();
    case kInE5M2: launch_backward_split<kInE5M2>(fixed, dyn, a, grid, stream); return hipGetLastError();
    default: break;
  }
  if (a.n <= small_batch_limit(3)) {
    launch_backward_split<kInF32>(fixed, dyn, a, grid, stream);
    return hipGetLastError();
  }
  const dim3 block(kWave);
  if (fixed) hipLaunchKernelGGL((sn::backward_kernel<true, false>), grid, block, 0, stream, a);
  else if (dyn) hipLaunchKernelGGL((sn::backward_kernel<false, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((sn::backward_kernel<false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_rotation_forward_small(const RotArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + sn::SPW - 1) / sn::SPW;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL((sn::rotation_forward_kernel<>), dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0, stream, a);
  return hipGetLastError();
}

}  // namespace bssm
