// Building blocks of the gfx950 kernels for the model shape of the Bayes
// layer: D = 4 key dims, M = 8 value columns
// (bayes_ssm/persistent_bayes_chunked_d4m8.cu is the reference extension for
// this shape; bayes_ssm/bayesian_layer.py:207-251 is the equation reference).
//
// Work decomposition: one wave64 per workgroup, 16 sequences per wave, a
// quad of 4 lanes per sequence.  Lane g of a quad owns covariance row g and
// value columns 2g, 2g+1 of the mean.  Everything a lane holds per row is
// stored *rotated*: slot m holds row (g + m) % 4, so
//   P[m]     = P[g][(g+m)%4]          Mv[m][c] = M[(g+m)%4][2g+c]
// and token vectors are read rotated from LDS (kr[m] = k[(g+m)%4]).  With
// that layout every cross-lane step is a single quad DPP rotation:
//   gather  (row values from their owners):  x_rot[m] = rot_m(x_g)
//   reduce-scatter (per-row partial sums):   x_g = x[0] + rot_3(x[1]) + rot_2(x[2]) + rot_1(x[3])
//   all-reduce (per-sequence scalars):       two xor DPP adds (bitwise identical in the quad)
// and the covariance stays bitwise symmetric, because entry (g, h) and its
// mirror (h, g) are computed by two lanes from commutative products only.
//
// Memory: all streamed tensors move through LDS tiles, addressed by
// per-workgroup buffer descriptors whose range ends at the last valid
// sequence, so rows past N read as zero and their stores are dropped without
// branches.  Tiles move whole cache lines of each sequence row (with
// nontemporal hints) and are laid out in LDS so that the per-token reads of
// 16 sequences are bank-conflict free (see Map).  A workgroup is a single
// wave, so LDS needs no barriers.
//
// Forward: 16-token tiles staged in registers (the next tile's loads are in
// flight while the current one is computed from LDS), so each sequence row
// is requested 256 bytes at a time.  Backward: the belief is checkpointed
// every 8 tokens; 16-token tiles (two checkpoint chunks) are staged in
// registers the same way (TileMap), and each chunk is replayed on chip
// (history in registers) and reversed from LDS while the next tile's loads
// are in flight; checkpoint records arrive by LDS-DMA (buffer_load ... lds).
// Checkpoints move as whole 16-byte pieces of each belief record (staged
// through LDS).

#pragma once

#include <type_traits>

#include "bssm_fp8.h"
#include "bssm_step.h"

namespace bssm {
namespace r4 {

constexpr int SPW = 16;   // sequences per wave
constexpr int TT = 8;     // forward tile, tokens
constexpr int SUB = 8;    // backward checkpoint chunk, tokens
constexpr int kDword3 = 0x00020000;  // raw fp32 buffer, gfx9 family
constexpr uint32_t kOob = 0x80000000u;  // offset past every descriptor range: load 0, drop store
// Cache policies: token streams and checkpoints are loaded and stored with
// the nontemporal hint (each byte moves once), except the 32- and 64-byte
// row pieces (p, r and their gradients, covariance records), which stay
// cached so that partial lines are merged before they reach HBM.  Streamed
// stores also carry the system-scope bit (sc1): at config 3 the step runs
// 8-9 us faster with it (D2M8 12 us; D8M8 and small batches unchanged; the
// same bit on loads changes nothing), consistent with the stores no longer
// displacing, in the 256 MB Infinity Cache, the lines the next kernel reads
// first.
constexpr bool kNtLoad = true;
constexpr int kStoreNt = 18;  // gfx940+ cache policy bits: nt (2) | sc1 (16)
constexpr int kNtStore = kStoreNt;
constexpr bool kNtCkpt = true;
// Tokens are separated by scheduling barriers (forward: every two tokens;
// backward: every replayed and every reversed token), and each token's
// look-ahead LDS reads are fenced right after their issue: without that
// fence the scheduler sinks those reads to the end of the previous token's
// region, and the token that consumes them waits out the whole LDS latency.

typedef float v2f __attribute__((ext_vector_type(2)));
using Rsrc = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ Rsrc make_rsrc(const float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, static_cast<int>(bytes), kDword3);
}

// 64 lanes x 16 bytes from global (voff + soff) into LDS at lds + 16 * lane.
// Issued as inline assembly on purpose: the compiler's own LDS-DMA tracking
// records a 16-byte footprint at `lds` and would let reads of the rest of
// the block run ahead of the data.  These loads are invisible to the
// compiler; their completion is awaited explicitly with vm_wait().
// The whole offset goes in the VGPR operand so that the descriptor's range
// check covers it (the scalar offset is outside the check on gfx9).
// NT = nontemporal (streamed once): used for streams whose DMA rows are
// whole 128-byte lines.
template <bool NT = false>
__device__ __forceinline__ void dma16(Rsrc r, const float* lds, uint32_t voff) {
  const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :
                 : "s"(base), "v"(voff), "s"(r)
                 : "memory");
  else
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(base), "v"(voff), "s"(r)
                 : "memory");
}

// Wait until at most N vector-memory operations are outstanding.  Loads
// complete in issue order among themselves (stores may overtake them), so
// N = the number of loads issued after the one awaited is always safe.
// The builtin keeps the compiler's own wait bookkeeping informed; the empty
// asm statements stop LDS reads from moving across the wait.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8.
  constexpr int kImm = (N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8);
  asm volatile("" : : : "memory");
  __builtin_amdgcn_s_waitcnt(kImm);
  asm volatile("" : : : "memory");
}

// Wait until every LDS operation of the wave has completed.
__device__ __forceinline__ void lds_wait() {
  asm volatile("" : : : "memory");
  __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));
  asm volatile("" : : : "memory");
}

// The raw buffer builtins move untyped 32-bit words; floats are bit-cast.
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
// AUX = cache-policy bits of the store (kStoreNt: nontemporal).
template <int AUX = 0>
__device__ __forceinline__ void st128(Rsrc r, v4f x, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, x), r, static_cast<int>(voff),
                                         static_cast<int>(soff), AUX);
}
__device__ __forceinline__ void st64(Rsrc r, v2f x, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, x), r, static_cast<int>(voff),
                                        static_cast<int>(soff), 0);
}
__device__ __forceinline__ void st32(Rsrc r, float x, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), r, static_cast<int>(voff),
                                        static_cast<int>(soff), 0);
}
__device__ __forceinline__ v2f ld64(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(voff),
                                                                      static_cast<int>(soff), 0));
}
__device__ __forceinline__ float ld32(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff),
                                                                        static_cast<int>(soff), 0));
}

// Value held by lane (g + R) % 4 of the caller's quad.
template <int R>
__device__ __forceinline__ float rot(float x) {
  constexpr int a = R & 3, b = (R + 1) & 3, c = (R + 2) & 3, d = (R + 3) & 3;
  return dpp<quad_perm(a, b, c, d)>(x);
}

// Sum over the quad; identical bits in all four lanes.
__device__ __forceinline__ float quad_sum(float x) {
  x += dpp<kXor1>(x);
  return x + dpp<kXor2>(x);
}

// Row-g total of a rotated per-row partial vector (slot m = row (g+m)%4).
__device__ __forceinline__ float reduce_scatter(const float (&x)[4]) {
  return ((x[0] + rot<3>(x[1])) + rot<2>(x[2])) + rot<1>(x[3]);
}

struct Bel {
  float P[4];      // P[g][(g+m)%4]
  float Mv[4][2];  // M[(g+m)%4][2g+c]
};

// Byte offsets of this lane's rotated belief entries inside one belief
// record of a sequence ([D, M] mean, [D, D] covariance, row-major).
struct BelOff {
  uint32_t m[4], c[4];
  __device__ __forceinline__ BelOff(int s, int g, uint32_t mean_stride, uint32_t cov_stride) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int row = (g + k) & 3;
      m[k] = static_cast<uint32_t>(s) * mean_stride + row * 32 + g * 8;
      c[k] = static_cast<uint32_t>(s) * cov_stride + g * 16 + row * 4;
    }
  }
};

__device__ __forceinline__ void load_bel(Bel& b, Rsrc rm, Rsrc rc, const BelOff& o, uint32_t soff_m,
                                         uint32_t soff_c) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    b.P[k] = ld32(rc, o.c[k], soff_c);
    const v2f x = ld64(rm, o.m[k], soff_m);
    b.Mv[k][0] = x[0];
    b.Mv[k][1] = x[1];
  }
}

__device__ __forceinline__ void store_bel(const Bel& b, Rsrc rm, Rsrc rc, const BelOff& o, uint32_t soff_m,
                                          uint32_t soff_c) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    st32(rc, b.P[k], o.c[k], soff_c);
    v2f x;
    x[0] = b.Mv[k][0];
    x[1] = b.Mv[k][1];
    st64(rm, x, o.m[k], soff_m);
  }
}

// A block of 16 belief records in LDS, natural layout: means [16][4][8] at
// float 0, covariances [16][4][4] at float 512.  Used to move checkpoints
// between registers (rotated) and memory (whole 16-byte pieces of each
// record, so every store or load covers its record contiguously).
constexpr int kRecFloats = 768;
__device__ __forceinline__ void bel_to_lds(const Bel& b, float* rec, int s, int g) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int row = (g + m) & 3;
    v2f x;
    x[0] = b.Mv[m][0];
    x[1] = b.Mv[m][1];
    *reinterpret_cast<v2f*>(&rec[s * 32 + row * 8 + 2 * g]) = x;
    rec[512 + s * 16 + g * 4 + row] = b.P[m];
  }
}
__device__ __forceinline__ void bel_from_lds(Bel& b, const float* rec, int s, int g) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int row = (g + m) & 3;
    const v2f x = *reinterpret_cast<const v2f*>(&rec[s * 32 + row * 8 + 2 * g]);
    b.Mv[m][0] = x[0];
    b.Mv[m][1] = x[1];
    b.P[m] = rec[512 + s * 16 + g * 4 + row];
  }
}
// Lane offsets of the 16-byte pieces of a record block: piece 64 j + lane of
// the means (j = 0, 1) and piece lane of the covariances, for records
// `mean_stride` / `cov_stride` bytes apart in memory.
struct RecOff {
  uint32_t m0, m1, c;
  __device__ __forceinline__ RecOff(int lane, uint32_t mean_stride, uint32_t cov_stride) {
    m0 = static_cast<uint32_t>(lane >> 3) * mean_stride + (lane & 7) * 16;
    m1 = static_cast<uint32_t>((64 + lane) >> 3) * mean_stride + (lane & 7) * 16;
    c = static_cast<uint32_t>(lane >> 2) * cov_stride + (lane & 3) * 16;
  }
};

// Token inputs of one lane (rotated vectors).
struct Tok {
  float kr[4], dr[4];
  float v[2];
  float p, r;
};

struct StepOut {
  float ug;    // u_g = (P' k)_g
  float s;     // unclamped innovation variance r + k.u
  float e[2];  // innovations of the own columns
};

// One token of the recurrence on the rotated belief.  u = P' k is computed
// as d * (P (d * k)) + p k; s = r + k.u is an all-reduce over the quad.
__device__ __forceinline__ void forward_step(Bel& b, const Tok& in, float floor, StepOut& o) {
  float wk[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) wk[m] = in.dr[m] * in.kr[m];
  float z = b.P[0] * wk[0];
#pragma unroll
  for (int m = 1; m < 4; ++m) z = fmaf(b.P[m], wk[m], z);
  const float ug = fmaf(in.dr[0], z, in.p * in.kr[0]);
  const float s = quad_sum(in.kr[0] * ug) + in.r;
  const float beta = fast_rcp(fmaxf(s, floor));
  float ur[4];
  ur[0] = ug;
  ur[1] = rot<1>(ug);
  ur[2] = rot<2>(ug);
  ur[3] = rot<3>(ug);
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float e = in.v[c];
#pragma unroll
    for (int m = 0; m < 4; ++m) e = fmaf(-b.Mv[m][c], wk[m], e);
    o.e[c] = e;
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float bu = beta * ur[m];
#pragma unroll
    for (int c = 0; c < 2; ++c) b.Mv[m][c] = fmaf(bu, o.e[c], in.dr[m] * b.Mv[m][c]);
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    float dp = (in.dr[0] * in.dr[m]) * b.P[m];
    if (m == 0) dp += in.p;
    b.P[m] = fmaf(-beta, ug * ur[m], dp);
  }
  o.ug = ug;
  o.s = s;
}

// Replay history of one token (everything the reverse needs that is not a
// token input): the belief before the token and the step intermediates.
struct Hist {
  float Pp[4];
  float Mp[4][2];
  float ug, s, e[2];
};

struct RevTok {
  float kr[4], dr[4], qr[4];
  float gy[2];
  float p;
};

struct RevOut {
  float gk, gq, gd, gp, gr;
  float gv[2];
  float gu;  // dL/du_g of the token
};

// Reverse of one token.  Carried adjoints (rotated like the belief):
// gM = dL/dM (own columns) and S = sym(dL/dP) (own row), updated in place to
// their values before the token.  With dL/dM_new including q gy^T:
//   ge = beta gM^T u (= dL/dv),  a = gM e,  w = S u,  z = u.(a - w)
//   gs = (s > floor) ? -z beta^2 : 0 (= dL/dr)
//   gu = beta (a - 2 w) + gs k
//   dL/dk = -d*(M_prev ge) + gs u + P' gu,   dL/dq = M_new gy = d*(M_prev gy) + beta u (e.gy)
// (M_new: the mean after the token, own columns, rotated like the belief).
//   H = S + sym(gu k^T),  dL/dd_i = 2 sum_j H_ij d_j P_ij + sum_c (gM - k ge^T)_ic M_prev_ic
//   dL/dp = trace(H),  S_prev = H * d d^T,  gM_prev = (gM - k ge^T) * d
template <bool DYN>
__device__ __forceinline__ void reverse_step(const RevTok& in, const Hist& h, const float (&Mn)[4][2],
                                             float (&gM)[4][2], float (&S)[4], float floor, RevOut& o) {
  const float beta = fast_rcp(fmaxf(h.s, floor));
  float ur[4];
  ur[0] = h.ug;
  ur[1] = rot<1>(h.ug);
  ur[2] = rot<2>(h.ug);
  ur[3] = rot<3>(h.ug);
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int c = 0; c < 2; ++c) gM[m][c] = fmaf(in.qr[m], in.gy[c], gM[m][c]);
  float ge[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float z = gM[0][c] * ur[0];
#pragma unroll
    for (int m = 1; m < 4; ++m) z = fmaf(gM[m][c], ur[m], z);
    ge[c] = beta * z;
    o.gv[c] = ge[c];
  }
  float av[4], Av[4], Cv[4], Bv[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    av[m] = fmaf(gM[m][1], h.e[1], gM[m][0] * h.e[0]);
    Av[m] = fmaf(h.Mp[m][1], ge[1], h.Mp[m][0] * ge[0]);
    Cv[m] = fmaf(Mn[m][1], in.gy[1], Mn[m][0] * in.gy[0]);
    float gb[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      gb[c] = fmaf(-in.kr[m], ge[c], gM[m][c]);
      gM[m][c] = gb[c] * in.dr[m];
    }
    Bv[m] = DYN ? fmaf(gb[1], h.Mp[m][1], gb[0] * h.Mp[m][0]) : 0.f;
  }
  const float a_g = reduce_scatter(av);
  const float A_g = reduce_scatter(Av);
  const float C_g = reduce_scatter(Cv);
  o.gq = C_g;

  float w = S[0] * ur[0];
#pragma unroll
  for (int m = 1; m < 4; ++m) w = fmaf(S[m], ur[m], w);
  const float z = quad_sum(h.ug * (a_g - w));
  const float gs = (h.s > floor) ? -z * beta * beta : 0.f;
  const float gu = fmaf(beta, fmaf(-2.f, w, a_g), gs * in.kr[0]);
  float gur[4];
  gur[0] = gu;
  gur[1] = rot<1>(gu);
  gur[2] = rot<2>(gu);
  gur[3] = rot<3>(gu);
  float dd[4], gk = fmaf(-in.dr[0], A_g, gs * h.ug);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    dd[m] = in.dr[0] * in.dr[m];
    float pb = dd[m] * h.Pp[m];
    if (m == 0) pb += in.p;
    gk = fmaf(pb, gur[m], gk);
  }
  o.gk = gk;
  const float hg = 0.5f * gu, hk = 0.5f * in.kr[0];
  float gd = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float hs = fmaf(hg, in.kr[m], fmaf(gur[m], hk, S[m]));
    if (DYN) gd = fmaf(hs * in.dr[m], h.Pp[m], gd);
    if (m == 0) o.gp = DYN ? quad_sum(hs) : 0.f;
    S[m] = hs * dd[m];
  }
  o.gd = DYN ? fmaf(2.f, gd, reduce_scatter(Bv)) : 0.f;
  o.gr = DYN ? gs : 0.f;
  o.gu = gu;
}

// Adjoint of the initial covariance: the full (asymmetric) derivative with
// respect to the covariance entering the first token,
// (S_in + gu k^T) * d d^T (persistent_bayes_chunked_d4m8.cu:320-326),
// recovered from the carried S_out = (S_in + sym(gu k^T)) * d d^T that the
// reverse of that token leaves:  S_out + (gu k^T - sym(gu k^T)) * d d^T.
__device__ __forceinline__ void initial_cov_adjoint(const float (&S)[4], float gu, const float (&kr)[4],
                                                    const float (&dr)[4], float (&gc0)[4]) {
  float gur[4];
  gur[0] = gu;
  gur[1] = rot<1>(gu);
  gur[2] = rot<2>(gu);
  gur[3] = rot<3>(gu);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float asym = 0.5f * fmaf(gu, kr[m], -gur[m] * kr[0]);
    gc0[m] = fmaf(asym, dr[0] * dr[m], S[m]);
  }
}

// ------------------------------------------------------------------ forward
// Tile layout.  A tile holds 8 tokens of the 16 sequences of a wave for
// one stream with W floats per token, moved as 16-byte pieces; lane l of
// DMA/store instruction j moves LDS piece 64 j + l.  Each instruction covers
// whole row segments in memory -- 8 rows x 8 pieces (128 B) for W = 4,
// 4 rows x 16 pieces (256 B) for W = 8, 16 rows x 2 pieces for W = 1 -- so
// every sequence row is read and written back as whole cache lines.  The
// order of the pieces inside an instruction's block puts the 16 rows' pieces
// of one token in distinct LDS banks (two per bank for the 512-byte W = 8
// reads) and keeps every lane's read address an affine function of the
// token, so the unrolled token loop addresses LDS with immediate offsets:
//   W = 4, piece t of row s = 8 j + a (j < 2):   slot 8 (t ^ j) + a
//   W = 8, piece c of row s = 4 j + a (j < 4):   slot 4 (c ^ 2 j) + a
//   W = 1, piece c of row s:                     piece 2 s + c
// Map holds, per instruction, the lane's byte offset inside the stream's
// 16-row block (relative to token 0 of the tile) and the first token its
// piece carries (for the tail masks).
struct Map {
  uint32_t d4[2], d8[4], d1;
  int t4[2], t8[4], t1;
  __device__ __forceinline__ Map(int lane, uint32_t row4, uint32_t row8, uint32_t row1) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = (lane >> 3) ^ j, sr = 8 * j + (lane & 7);
      d4[j] = static_cast<uint32_t>(sr) * row4 + t * 16;
      t4[j] = t;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = (lane >> 2) ^ (2 * j), sr = 4 * j + (lane & 3);
      d8[j] = static_cast<uint32_t>(sr) * row8 + c * 16;
      t8[j] = c >> 1;
    }
    d1 = lane < 32 ? static_cast<uint32_t>(lane >> 1) * row1 + (lane & 1) * 16 : kOob;
    t1 = lane < 32 ? 4 * (lane & 1) : 1 << 20;
  }
};

// LDS float indices of one lane's reads inside a tile.  For sequence s and
// token tt (a compile-time constant in the unrolled loops):
//   W = 4: word w of the token   = 4 (64 j + 8 (p ^ j) + a) - 32 p + 32 tt + w,
//          j = s >> 3, a = s & 7, p = tt & 1
//   W = 8: own columns 2g, 2g+1  = 4 (64 j + 8 (c ^ j) + 4 (g >> 1) + a) + 2 (g & 1) + 128 (tt >> 2),
//          j = s >> 2, a = s & 3, c = tt & 3
//   W = 1: the token             = 8 s + tt
struct Idx {
  // Plain arithmetic on scalars: the token index is a run-time value in the
  // partial-tile loops, and any member chosen by it (an array element, or a
  // select between members, which the compiler turns into a computed address)
  // would force the whole per-lane core object out of registers.
  int w4a, d4, w8, j8, w1;
  __device__ __forceinline__ Idx(int s, int g) {
    const int j4 = s >> 3, a4 = s & 7;
    w4a = 4 * (64 * j4 + 8 * j4 + a4);  // parity 0; parity 1 is 64 j4 words lower
    d4 = -64 * j4;
    j8 = s >> 2;
    w8 = 4 * (64 * j8 + 4 * (g >> 1) + (s & 3)) + 2 * (g & 1);
    w1 = 8 * s;
  }
  __device__ __forceinline__ int i4(int tt, int w) const { return w4a + (tt & 1) * d4 + 32 * tt + w; }
  __device__ __forceinline__ int i8(int tt) const { return w8 + 32 * ((tt & 3) ^ j8) + 128 * (tt >> 2); }
  __device__ __forceinline__ int i1(int tt) const { return w1 + tt; }
};

// One forward tile holds 16 tokens of the 16 sequences as two 8-token
// sub-tiles in the layout above (floats per sub-tile): k, d, q [8 x 16 x 4],
// v [8 x 16 x 8] (values in, readouts out, in place), p and r [16 x 8].
struct FwdTile {
  static constexpr int K = 0, D = 512, Q = 1024, V = 1536, P = 2560, R = 2688, SIZE = 2816;
};
constexpr int LT = 2 * TT;  // tokens per register-staged load tile

// The per-token forward over one 8-token LDS sub-tile (FwdTile layout) and
// the checkpoint stores, shared by the forward kernels.  Holds the belief of
// the lane's row and the checkpoint schedule (a record before every token
// t0 + j * chunk, staged through LDS and stored as whole 16-byte pieces).
template <bool FIXED>
struct FwdCore {
  Bel b;
  Idx ix;
  int lane, g, s;
  float floor;
  int64_t chunk, next_ckpt;
  uint32_t ckpt;
  RecOff ckoff;
  float* ckst;  // LDS staging of one checkpoint record (kRecFloats)

  __device__ __forceinline__ FwdCore(int lane_, float floor_, int64_t chunk_, uint32_t nbp,
                                     float* ckst_)
      : ix(lane_ >> 2, lane_ & 3), lane(lane_), g(lane_ & 3), s(lane_ >> 2), floor(floor_), chunk(chunk_),
        next_ckpt(chunk_), ckpt(1), ckoff(lane_, nbp * 128u, nbp * 64u), ckst(ckst_) {}

  // Checkpoint record c of the 16 sequences.
  __device__ __forceinline__ void store_ckpt(uint32_t c, Rsrc rbm, Rsrc rbc) {
    bel_to_lds(b, ckst, s, g);
    const v4f x0 = *reinterpret_cast<const v4f*>(&ckst[lane * 4]);
    const v4f x1 = *reinterpret_cast<const v4f*>(&ckst[256 + lane * 4]);
    const v4f x2 = *reinterpret_cast<const v4f*>(&ckst[512 + lane * 4]);
    st128<kNtCkpt ? kStoreNt : 0>(rbm, x0, ckoff.m0, c * 128u);
    st128<kNtCkpt ? kStoreNt : 0>(rbm, x1, ckoff.m1, c * 128u);
    st128(rbc, x2, ckoff.c, c * 64u);
  }

  // Token inputs of one lane, read from LDS ahead of their use.
  struct In {
    Tok t;
    float qr[4];
  };
  __device__ __forceinline__ void read_in(const float* tl, int tt, In& x) const {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int e = ix.i4(tt, (g + m) & 3);
      x.t.kr[m] = (tl + FwdTile::K)[e];
      x.t.dr[m] = FIXED ? kFixedDecay : (tl + FwdTile::D)[e];
      x.qr[m] = (tl + FwdTile::Q)[e];
    }
    const v2f vv = *reinterpret_cast<const v2f*>(&(tl + FwdTile::V)[ix.i8(tt)]);
    x.t.v[0] = vv[0];
    x.t.v[1] = vv[1];
    x.t.p = FIXED ? kFixedProcess : (tl + FwdTile::P)[ix.i1(tt)];
    x.t.r = FIXED ? kFixedObservation : (tl + FwdTile::R)[ix.i1(tt)];
  }
  __device__ __forceinline__ void step(const In& x, v2f& y) {
    StepOut o;
    forward_step(b, x.t, floor, o);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float acc = b.Mv[0][c] * x.qr[0];
#pragma unroll
      for (int m = 1; m < 4; ++m) acc = fmaf(b.Mv[m][c], x.qr[m], acc);
      y[c] = acc;
    }
  }
  // Readouts overwrite the token's values in the V region.
  __device__ __forceinline__ void put_y(float* tl, int tt, v2f y) const {
    *reinterpret_cast<v2f*>(&(tl + FwdTile::V)[ix.i8(tt)]) = y;
  }
  // A full sub-tile: the LDS reads of tokens 2j+2 and 2j+3 are issued before
  // tokens 2j and 2j+1 are computed (the scheduling barrier keeps them
  // there), and the readouts stay in registers until the last token, so no
  // LDS write sits between reads.
  __device__ __forceinline__ void full_tile(float* tl) {
    In x[TT];
    v2f y[TT];
    read_in(tl, 0, x[0]);
    read_in(tl, 1, x[1]);
#pragma unroll
    for (int j = 0; j < TT / 2; ++j) {
      if (j + 1 < TT / 2) {
        read_in(tl, 2 * j + 2, x[2 * j + 2]);
        read_in(tl, 2 * j + 3, x[2 * j + 3]);
        __builtin_amdgcn_sched_barrier(0);
      }
      step(x[2 * j], y[2 * j]);
      step(x[2 * j + 1], y[2 * j + 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) put_y(tl, tt, y[tt]);
  }
  // Sub-tile starting at token t0 (fewer than TT tokens at the end of T).
  __device__ __forceinline__ void run_sub(float* tl, int64_t t0, int64_t T, Rsrc rbm, Rsrc rbc) {
    const int len = static_cast<int>((T - t0) < TT ? (T - t0) : TT);
    if (t0 == next_ckpt) {
      store_ckpt(ckpt, rbm, rbc);
      ++ckpt;
      next_ckpt += chunk;
    }
    if (len == TT && next_ckpt >= t0 + TT) {
      full_tile(tl);
    } else {
#pragma unroll 1
      for (int tt = 0; tt < len; ++tt) {
        if (t0 + tt == next_ckpt) {
          store_ckpt(ckpt, rbm, rbc);
          ++ckpt;
          next_ckpt += chunk;
        }
        In x;
        v2f y;
        read_in(tl, tt, x);
        step(x, y);
        put_y(tl, tt, y);
      }
    }
  }
};

// 16-byte load of one lane's piece (voff carries the whole offset so that
// the descriptor's range check covers it).
template <bool NT>
__device__ __forceinline__ v4f ld128(Rsrc r, uint32_t voff) {
  return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), 0, NT ? 2 : 0));
}
// The same with a uniform part in the scalar offset, which the range check
// does not cover: voff must carry the row, and the caller keeps the piece
// inside its row (or passes kOob, which drops it).
template <bool NT>
__device__ __forceinline__ v4f ld128(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff),
                                                                       static_cast<int>(soff), NT ? 2 : 0));
}

// Register staging of one 16-token forward tile: for each sub-tile h and
// DMA-shaped instruction j, the lane's piece (the same pieces the Map
// describes, so every instruction still moves whole row segments and the two
// halves of a row are requested back to back).  p and r take one
// instruction each: lane l -> row l >> 2, piece l & 3 (16 rows x 64 B).
struct FwdStage {
  v4f k[4], q[4], d[4], v[8], p, r;
};
// With bf16 keys, queries and values (H): the bf16 pieces of the maps in
// HalfMap, widened into the same float32 slots when written to LDS.
struct FwdStageH {
  v4f k[2], q[2], d[4], v[4], p, r;
};

__device__ __forceinline__ const float* byte_offset(const float* p, int64_t bytes) {
  return reinterpret_cast<const float*>(reinterpret_cast<const char*>(p) + bytes);
}

// bf16 pairs (low half first) to float32, and back with round to nearest even.
__device__ __forceinline__ v4f widen_lo(v4f piece) {
  const v4u w = __builtin_bit_cast(v4u, piece);
  v4f out;
  out[0] = __builtin_bit_cast(float, w[0] << 16);
  out[1] = __builtin_bit_cast(float, w[0] & 0xffff0000u);
  out[2] = __builtin_bit_cast(float, w[1] << 16);
  out[3] = __builtin_bit_cast(float, w[1] & 0xffff0000u);
  return out;
}
__device__ __forceinline__ v4f widen_hi(v4f piece) {
  const v4u w = __builtin_bit_cast(v4u, piece);
  v4f out;
  out[0] = __builtin_bit_cast(float, w[2] << 16);
  out[1] = __builtin_bit_cast(float, w[2] & 0xffff0000u);
  out[2] = __builtin_bit_cast(float, w[3] << 16);
  out[3] = __builtin_bit_cast(float, w[3] & 0xffff0000u);
  return out;
}
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t narrow2(float x, float y) {
  bf2 v;
  v[0] = static_cast<__bf16>(x);
  v[1] = static_cast<__bf16>(y);
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ v4f narrow(v4f lo, v4f hi) {
  v4u w;
  w[0] = narrow2(lo[0], lo[1]);
  w[1] = narrow2(lo[2], lo[3]);
  w[2] = narrow2(hi[0], hi[1]);
  w[3] = narrow2(hi[2], hi[3]);
  return __builtin_bit_cast(v4f, w);
}

// Per-lane maps of the bf16 streams of a 16-token tile (16-byte pieces):
//   k, q: row 8I + (l & 7), tokens t0 + 2 (l >> 3) and + 1 (I < 2)
//   v:    row 4I + (l & 3), token t0 + (l >> 2) (I < 4)
// with their global byte offsets and the LDS float offsets (relative to the
// K or Q region, and to the V region, of an 8-token slot of slot_floats) of
// the two widened float32 pieces each becomes, in the float32 slot layout.
struct HalfMap {
  int k_lds[2][2], v_lds[4][2];
  uint32_t k_off[2], v_off[4];
  int k_tok, v_tok;  // first token of the lane's piece within the tile
  __device__ __forceinline__ HalfMap(int lane, int slot_floats, uint32_t row4h, uint32_t row8h) {
    const int pc = lane >> 3, a8 = lane & 7;
    k_tok = 2 * pc;
#pragma unroll
    for (int I = 0; I < 2; ++I) {
      k_off[I] = static_cast<uint32_t>(8 * I + a8) * row4h + static_cast<uint32_t>(pc) * 16u;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int tok = k_tok + e, tt = tok & 7;
        k_lds[I][e] = (tok >> 3) * slot_floats + 4 * (64 * I + 8 * (tt ^ I) + a8);
      }
    }
    const int tv = lane >> 2, a4 = lane & 3;
    v_tok = tv;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      v_off[I] = static_cast<uint32_t>(4 * I + a4) * row8h + static_cast<uint32_t>(tv) * 16u;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int c = 2 * (tv & 7) + e;
        v_lds[I][e] = (tv >> 3) * slot_floats + 4 * (64 * I + 4 * (c ^ (2 * I)) + a4);
      }
    }
  }
};

// Per-lane maps of the float8 streams of a 16-token tile (16-byte pieces):
//   k, q: row l >> 2, tokens t0 + 4 (l & 3) .. + 3
//   v:    row 8I + (l >> 3), tokens t0 + 2 (l & 7) and + 1 (I < 2)
// Each 32-bit word of a piece is one token's 4 key values (k, q; word u is
// token k_tok + u) or half of a token's 8 values (v; word w is token
// v_tok + (w >> 1), values 4 (w & 1) .. + 3).  k_lds / v_lds are the LDS
// float offsets of the float32 piece each word becomes, in HalfMap's slot
// layout; a row's 64 (k, q) or 128 (v) bytes of the tile are read by 4 or 8
// consecutive lanes.
struct QuarterMap {
  int k_lds[4], v_lds[2][4];
  uint32_t k_off, v_off[2];
  int k_tok, v_tok;  // first token of the lane's pieces within the tile
  __device__ __forceinline__ QuarterMap(int lane, int slot_floats, uint32_t row4q, uint32_t row8q) {
    const int kr = lane >> 2, pc = lane & 3, ki = kr >> 3, k8 = kr & 7;
    k_tok = 4 * pc;
    k_off = static_cast<uint32_t>(kr) * row4q + static_cast<uint32_t>(pc) * 16u;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tok = k_tok + u, tt = tok & 7;
      k_lds[u] = (tok >> 3) * slot_floats + 4 * (64 * ki + 8 * (tt ^ ki) + k8);
    }
    const int tp = lane & 7;
    v_tok = 2 * tp;
#pragma unroll
    for (int I = 0; I < 2; ++I) {
      const int vr = 8 * I + (lane >> 3), vi = vr >> 2, a4 = vr & 3;
      v_off[I] = static_cast<uint32_t>(vr) * row8q + static_cast<uint32_t>(tp) * 16u;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int tok = v_tok + (w >> 1), c = 2 * (tok & 7) + (w & 1);
        v_lds[I][w] = (tok >> 3) * slot_floats + 4 * (64 * vi + 4 * (c ^ (2 * vi)) + a4);
      }
    }
  }
};
// Register staging of a forward tile with float8 keys, queries and values.
struct FwdStageQ {
  v4f k, q, d[4], v[2], p, r;
};

// ----------------------------------------------------------------- backward
// One backward chunk slot (floats): k, d, q [8 x 16 x 4] (inputs, then their
// gradients in place), v [8 x 16 x 8] (values, then value gradients), gy
// [8 x 16 x 8], p and r [16 x 8 used] (inputs, then gradients), and the
// chunk's checkpoint (belief records, natural layout).
struct BwdTile {
  static constexpr int K = 0, D = 512, Q = 1024, V = 1536, GY = 2560, P = 3584, R = 3840, CK = 4096,
                       SIZE = 4096 + kRecFloats;
};

// Per-lane maps of the float32 streams of a 16-token backward tile (two
// BwdTile slots), staged through registers.  Every load or store
// instruction covers whole 16-token row segments -- the 256 (W = 4), 512
// (W = 8) or 64 (W = 1) bytes of a sequence row in one instruction -- which
// measured 11 % faster on this access mix than 8-token (128-byte) pieces and
// 6 % faster than the same 256 bytes split over two instructions:
//   W = 4 (k, d, q and their gradients): instruction I < 4: row 4I + (l >> 4), token l & 15
//   W = 8 (v, gy, dL/dv):                instruction I < 8: row 2I + (l >> 5), piece l & 31
//                                        (token (l & 31) >> 1, values 4 (l & 1) .. + 3)
//   W = 1 (p, r and their gradients):    row l >> 2, tokens 4 (l & 3) .. + 3
// o*: byte offset of the lane's piece from the row block's first token of
// the tile; s*: float offset of the piece in the two-slot LDS tile (each
// slot in the BwdTile layout, addressed per token by Idx); t*: the piece's
// first token within the tile.
struct TileMap {
  uint32_t o4[4], o8[8], o1;
  int s4[4], s8[8], s1;
  int t4, t8, t1;
  __device__ __forceinline__ TileMap(int lane, uint32_t row4, uint32_t row8, uint32_t row1) {
    t4 = lane & 15;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int s = 4 * I + (lane >> 4), j = s >> 3, a = s & 7, t = t4 & 7;
      o4[I] = static_cast<uint32_t>(s) * row4 + static_cast<uint32_t>(t4) * 16u;
      s4[I] = (t4 >> 3) * BwdTile::SIZE + 4 * (64 * j + 8 * (t ^ j) + a);
    }
    const int c16 = lane & 31;
    t8 = c16 >> 1;
#pragma unroll
    for (int I = 0; I < 8; ++I) {
      const int s = 2 * I + (lane >> 5), j = s >> 2, a = s & 3, c = 2 * (t8 & 7) + (c16 & 1);
      o8[I] = static_cast<uint32_t>(s) * row8 + static_cast<uint32_t>(c16) * 16u;
      s8[I] = (t8 >> 3) * BwdTile::SIZE + 4 * (64 * j + 4 * (c ^ (2 * j)) + a);
    }
    t1 = 4 * (lane & 3);
    o1 = static_cast<uint32_t>(lane >> 2) * row1 + static_cast<uint32_t>(lane & 3) * 16u;
    s1 = ((lane & 3) >> 1) * BwdTile::SIZE + 4 * (2 * (lane >> 2) + (lane & 1));
  }
};

// Replay and reverse of one checkpoint chunk held in a BwdTile slot, and the
// adjoints carried across chunks (shared by the backward kernels).
template <bool FIXED, bool DYN>
struct BwdCore {
  Idx ix;
  int g;
  float floor;
  float gM[4][2], S[4];
  // Token 0 of the chunk reversed last: the sequence's first token once the
  // whole sequence has been reversed (for the initial-covariance adjoint).
  float first_gu, first_kr[4], first_dr[4];

  __device__ __forceinline__ BwdCore(int s, int g_, float floor_) : ix(s, g_), g(g_), floor(floor_) {}

  // Carried adjoints from the final-state gradients gmf, gcf (null = zero;
  // `any` is any valid device address, used as a base of an empty range).
  __device__ __forceinline__ void init(const float* gmf, const float* gcf, const float* any, int64_t n0,
                                       uint32_t valid, const BelOff& unit, int s) {
    const bool has_m = gmf != nullptr, has_c = gcf != nullptr;
    const Rsrc rgm = make_rsrc(has_m ? gmf + n0 * 32 : any, has_m ? valid * 128u : 0u);
    const Rsrc rgc = make_rsrc(has_c ? gcf + n0 * 16 : any, has_c ? valid * 64u : 0u);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const v2f x = ld64(rgm, unit.m[m], 0);
      gM[m][0] = x[0];
      gM[m][1] = x[1];
      // Mirror entry (row (g+m)%4, column g) sits at the transposed offset.
      const int h = (g + m) & 3;
      const uint32_t tr = static_cast<uint32_t>(s) * 64u + h * 16 + g * 4;
      S[m] = 0.5f * (ld32(rgc, unit.c[m], 0) + ld32(rgc, tr, 0));
    }
  }
  // Adjoints of the initial mean and covariance (null: not requested).
  __device__ __forceinline__ void store_initial(float* gm0_out, float* gc0_out, int64_t n0, uint32_t valid,
                                                const BelOff& unit) const {
    if (gm0_out) {
      const Rsrc rgm0 = make_rsrc(gm0_out + n0 * 32, valid * 128u);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        v2f x;
        x[0] = gM[m][0];
        x[1] = gM[m][1];
        st64(rgm0, x, unit.m[m], 0);
      }
    }
    if (gc0_out) {
      float gc0[4];
      initial_cov_adjoint(S, first_gu, first_kr, first_dr, gc0);
      const Rsrc rgc0 = make_rsrc(gc0_out + n0 * 16, valid * 64u);
#pragma unroll
      for (int m = 0; m < 4; ++m) st32(rgc0, gc0[m], unit.c[m], 0);
    }
  }

  __device__ __forceinline__ void read_tok(const float* tl, int tt, Tok& in) const {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int e = ix.i4(tt, (g + m) & 3);
      in.kr[m] = (tl + BwdTile::K)[e];
      in.dr[m] = FIXED ? kFixedDecay : (tl + BwdTile::D)[e];
    }
    const v2f vv = *reinterpret_cast<const v2f*>(&(tl + BwdTile::V)[ix.i8(tt)]);
    in.v[0] = vv[0];
    in.v[1] = vv[1];
    in.p = FIXED ? kFixedProcess : (tl + BwdTile::P)[ix.i1(tt)];
    in.r = FIXED ? kFixedObservation : (tl + BwdTile::R)[ix.i1(tt)];
  }
  __device__ __forceinline__ void read_rev(const float* tl, int tt, RevTok& in) const {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int e = ix.i4(tt, (g + m) & 3);
      in.kr[m] = (tl + BwdTile::K)[e];
      in.dr[m] = FIXED ? kFixedDecay : (tl + BwdTile::D)[e];
      in.qr[m] = (tl + BwdTile::Q)[e];
    }
    const v2f gyv = *reinterpret_cast<const v2f*>(&(tl + BwdTile::GY)[ix.i8(tt)]);
    in.gy[0] = gyv[0];
    in.gy[1] = gyv[1];
    in.p = FIXED ? kFixedProcess : (tl + BwdTile::P)[ix.i1(tt)];
  }
  __device__ __forceinline__ void replay(Bel& b, const Tok& in, Hist& h) const {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      h.Pp[m] = b.P[m];
      h.Mp[m][0] = b.Mv[m][0];
      h.Mp[m][1] = b.Mv[m][1];
    }
    StepOut o;
    forward_step(b, in, floor, o);
    h.ug = o.ug;
    h.s = o.s;
    h.e[0] = o.e[0];
    h.e[1] = o.e[1];
  }
  __device__ __forceinline__ void reverse(float* tl, int tt, const RevTok& in, const Hist& h,
                                         const float (&Mn)[4][2]) {
    RevOut o;
    reverse_step<DYN>(in, h, Mn, gM, S, floor, o);
    if (tt == 0) {
      first_gu = o.gu;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        first_kr[m] = in.kr[m];
        first_dr[m] = in.dr[m];
      }
    }
    const int ow = ix.i4(tt, g);  // own-row word of the token's piece
    (tl + BwdTile::K)[ow] = o.gk;
    (tl + BwdTile::Q)[ow] = o.gq;
    (tl + BwdTile::D)[ow] = o.gd;
    v2f gv;
    gv[0] = o.gv[0];
    gv[1] = o.gv[1];
    *reinterpret_cast<v2f*>(&(tl + BwdTile::V)[ix.i8(tt)]) = gv;
    (tl + BwdTile::P)[ix.i1(tt)] = o.gp;
    (tl + BwdTile::R)[ix.i1(tt)] = o.gr;
  }
  // Replay the chunk from its checkpoint, then reverse it; gradients
  // overwrite the chunk's input tiles.  Tokens are separated by scheduling
  // barriers, and each token's LDS reads are issued one token ahead (the
  // reads of the first reverse token during the last replay token), in
  // program order before the gradient writes that follow them.
  template <int LEN>
  __device__ __forceinline__ void process(float* tl, Bel& b) {
    Hist h[LEN];
    Tok x[LEN];
    RevTok rx[LEN];
    read_tok(tl, 0, x[0]);
#pragma unroll
    for (int tt = 0; tt < LEN; ++tt) {
      if (tt + 1 < LEN) read_tok(tl, tt + 1, x[tt + 1]);
      else read_rev(tl, LEN - 1, rx[LEN - 1]);
      __builtin_amdgcn_sched_barrier(0);
      replay(b, x[tt], h[tt]);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int tt = LEN - 1; tt >= 0; --tt) {
      if (tt > 0) read_rev(tl, tt - 1, rx[tt - 1]);
      __builtin_amdgcn_sched_barrier(0);
      // The mean after token tt: the next token's history, or the replayed
      // belief after the chunk's last token.
      reverse(tl, tt, rx[tt], h[tt], tt + 1 < LEN ? h[tt + 1 < LEN ? tt + 1 : tt].Mp : b.Mv);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Advance the belief over the 8 tokens of a slot without keeping history
  // (the start of a tile's second chunk when one record covers 16 tokens).
  __device__ __forceinline__ void advance(const float* tl, Bel& b) const {
    Tok x[SUB];
    read_tok(tl, 0, x[0]);
#pragma unroll
    for (int tt = 0; tt < SUB; ++tt) {
      if (tt + 1 < SUB) read_tok(tl, tt + 1, x[tt + 1]);
      __builtin_amdgcn_sched_barrier(0);
      StepOut o;
      forward_step(b, x[tt], floor, o);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // A chunk of `len` tokens (SUB, or 4 for the last one of T = 8n + 4).
  __device__ __forceinline__ void run(float* tl, Bel& b, int len) {
    if (len == SUB) process<SUB>(tl, b);
    else process<4>(tl, b);
  }
};

}  // namespace r4
}  // namespace bssm
