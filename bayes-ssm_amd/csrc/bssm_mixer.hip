// Producer-fused D = 4, M = 8 layer core of the Bayes mixer, gfx950.
//
// The mixer (example/train_6layer.py:613-729, learned dynamics) turns its
// bfloat16 projections into the layer inputs per (batch b, token t, head h):
//   q, k = normalize(silu(q_proj), silu(k_proj))    (per-head L2, eps 1e-12)
//   v = silu(v_proj),  d = exp(-softplus(decay_logits)),
//   p = softplus(noise[.., 0]) + 1e-4,  r = softplus(noise[.., 1]) + 1e-4
// then permutes [B, T, H, .] to the layer's [B * H, T, .] rows, runs the
// recurrence, and permutes the readout back to [B, T, H, 8].  Here all of it
// happens in the recurrence kernels: a wave takes 16 consecutive heads of one
// batch row, whose per-token slices are contiguous in the [B, T, H, .]
// tensors (128 bytes of keys, 256 of values), so every projection is read
// once, in place, and widened, transformed and written into the float32 LDS
// slot layout of bssm_rot4.h at the tile's staging; the readout leaves the
// same way.  The transforms run in float32 on the widened bf16 values (the
// reference computes them in float32 after .to(float32) unless its
// bf16_state_projection option is set).
//
// The backward stages the same raw pieces, keeps them in registers for the
// tile, and at the tile's write-out applies the chain rule of the
// transforms to the gradients the reverse leaves in LDS, so the projection
// gradients are written directly (bfloat16, or float32 for testing).
//
// Piece maps of a 16-token tile starting at t0 (lane l, instruction I):
//   q, k, decay logits (8 per token):  token 8I + (l >> 3), heads 2 (l & 7), +1
//   v (16 per token):                  token 4I + (l >> 4), head l & 15
//   noise (4 per token):               token l >> 2, heads 4 (l & 3) .. + 3
//   readout, gy (32 per token):        token 2I + (l >> 5), head (l >> 1) & 15, half l & 1
// Each map's rows are addressed through a per-batch-row buffer descriptor
// whose range ends at token T, so a partial last tile reads zeros and drops
// its stores without per-lane masks.

#include "bssm_rot4.h"

namespace bssm {
namespace r4 {
namespace {

constexpr float kNoiseFloor = 1e-4f;  // softplus(noise) + 1e-4 (train_6layer.py:667-668)
// F.normalize divides by max(|a|, 1e-12): 1 / max(|a|, eps) = min(rsq(|a|^2), 1e12).
constexpr float kInvNormEps = 1e12f;
constexpr float kNormEps2 = 1e-24f;

// The transforms run on the hardware exponential, reciprocal and reciprocal
// square root (v_exp_f32, v_rcp_f32, v_rsq_f32, each within 1 ulp, the
// exponential's argument scaled by log2 e first); the library logf/log1pf
// and the IEEE divide cost 13 to 117 instructions each.
__device__ __forceinline__ float exp_(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
__device__ __forceinline__ float rcp_(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float sigmoid_(float x) { return rcp_(1.f + exp_(-x)); }

// log(1 + u) for u in [0, 1]: 2 atanh(s) with s = u / (2 + u) <= 1/3, the
// odd series through s^15 (next term below 2e-9 relative).
__device__ __forceinline__ float log1p01(float u) {
  const float s = u * rcp_(2.f + u), z = s * s;
  float p = 1.f / 15.f;
  p = fmaf(p, z, 1.f / 13.f);
  p = fmaf(p, z, 1.f / 11.f);
  p = fmaf(p, z, 1.f / 9.f);
  p = fmaf(p, z, 1.f / 7.f);
  p = fmaf(p, z, 1.f / 5.f);
  p = fmaf(p, z, 1.f / 3.f);
  p = fmaf(p, z, 1.f);
  return 2.f * s * p;
}
// softplus(x) = max(x, 0) + log(1 + e^-|x|) and its derivative sigmoid(x).
// torch's softplus returns x itself above 20, where log(1 + e^-x) < 2.1e-9
// is below half an ulp of x, so the two agree.
__device__ __forceinline__ float softplus_(float x) { return fmaxf(x, 0.f) + log1p01(exp_(-fabsf(x))); }

// The decay exp(-softplus(z)) = 2^-(max(z, 0) log2 e + log2(1 + e^-|z|)),
// with the hardware log2: its absolute error (about 1e-7 in the exponent,
// from rounding 1 + e^-|z|) is one ulp of the decay, so the series of
// log1p01 (which the noise needs for its relative accuracy where softplus is
// tiny) is not needed here.
__device__ __forceinline__ float decay_(float z) {
  const float l = __builtin_amdgcn_logf(1.f + exp_(-fabsf(z)));
  return __builtin_amdgcn_exp2f(-fmaf(fmaxf(z, 0.f), 1.44269504088896341f, l));
}

// silu(x) = x sigmoid(x); silu'(x) = sigmoid(x) (1 + x (1 - sigmoid(x))).
__device__ __forceinline__ float silu_(float x) { return x * sigmoid_(x); }

// normalize(silu(x)) of one head's key or query vector.
__device__ __forceinline__ v4f unit_silu(v4f x) {
  v4f a;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = silu_(x[i]);
    ss = fmaf(a[i], a[i], ss);
  }
  return a * fminf(__builtin_amdgcn_rsqf(ss), kInvNormEps);
}
// Gradient through normalize(silu(x)): g is dL/d(output).  Above the eps
// clamp, d(a/|a|) = (g - w (w . g)) / |a| with w = a / |a|; below it the map
// is a / eps.
__device__ __forceinline__ v4f unit_silu_grad(v4f x, v4f g) {
  v4f a, ds;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float sg = sigmoid_(x[i]);
    a[i] = x[i] * sg;
    ds[i] = sg * fmaf(x[i], 1.f - sg, 1.f);
    ss = fmaf(a[i], a[i], ss);
  }
  const float rn = fminf(__builtin_amdgcn_rsqf(ss), kInvNormEps);
  float wg = 0.f;
  if (ss > kNormEps2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) wg = fmaf(a[i] * rn, g[i], wg);
  }
  v4f out;
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = fmaf(-a[i] * rn, wg, g[i]) * rn * ds[i];
  return out;
}

__device__ __forceinline__ const float* as_f(const void* p, int64_t bytes) {
  return reinterpret_cast<const float*>(reinterpret_cast<const char*>(p) + bytes);
}

// Per-lane piece offsets (bytes within a token row of the wave's heads, and
// the row index) and LDS float offsets of the maps above, for an 8-token slot
// layout of slot_floats floats.
struct MixMap {
  int kq_tok[2];        // token of the q/k/decay piece (within the tile)
  uint32_t kq_col;      // byte offset of the piece within the wave's q/k/decay slice
  int kq_lds[2][2];     // LDS offsets (relative to the region) of its two heads
  int v_tok[4];
  uint32_t v_col;
  int v_lds[4][2];      // the two halves (value columns 0-3, 4-7)
  int nz_tok;
  uint32_t nz_col;
  int nz_lds[4];        // P-region offsets of the piece's four heads (R: same + R - P)
  int y_tok[8];
  uint32_t y_col;
  int y_lds[8];

  __device__ __forceinline__ MixMap(int lane, int slot_floats) {
    const int pc = lane & 7;
#pragma unroll
    for (int I = 0; I < 2; ++I) {
      kq_tok[I] = 8 * I + (lane >> 3);
      const int tt = kq_tok[I] & 7, sub = kq_tok[I] >> 3;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int sq = 2 * pc + e, j = sq >> 3, a8 = sq & 7;
        kq_lds[I][e] = sub * slot_floats + 4 * (64 * j + 8 * (tt ^ j) + a8);
      }
    }
    kq_col = static_cast<uint32_t>(pc) * 16u;
    const int hh = lane & 15;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      v_tok[I] = 4 * I + (lane >> 4);
      const int tt = v_tok[I] & 7, sub = v_tok[I] >> 3, j = hh >> 2, a4 = hh & 3;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int c = 2 * tt + e;
        v_lds[I][e] = sub * slot_floats + 4 * (64 * j + 4 * (c ^ (2 * j)) + a4);
      }
    }
    v_col = static_cast<uint32_t>(hh) * 16u;
    nz_tok = lane >> 2;
    nz_col = static_cast<uint32_t>(lane & 3) * 16u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int sq = 4 * (lane & 3) + e;
      nz_lds[e] = (nz_tok >> 3) * slot_floats + 8 * sq + (nz_tok & 7);
    }
    const int yh = (lane >> 1) & 15, half = lane & 1;
#pragma unroll
    for (int I = 0; I < 8; ++I) {
      y_tok[I] = 2 * I + (lane >> 5);
      const int tt = y_tok[I] & 7, sub = y_tok[I] >> 3, j = yh >> 2, a4 = yh & 3, c = 2 * tt + half;
      y_lds[I] = sub * slot_floats + 4 * (64 * j + 4 * (c ^ (2 * j)) + a4);
    }
    y_col = static_cast<uint32_t>(yh) * 32u + static_cast<uint32_t>(half) * 16u;
  }
};

// Raw projection pieces of one 16-token tile.
struct MixRaw {
  v4f q[2], k[2], dl[2], v[4], nz;
};

// The aux bias of the wave's 16 heads, staged in LDS at the kernel's start
// (slot pc < 8: the decay-logit piece of lane pc's columns, slot 8 + j: the
// noise piece of lane j's columns, 8 bf16 each), added to a tile's raw
// decay-logit and noise pieces before they are used: bf16(x + b), rounded
// to nearest even once, as torch adds two bf16 tensors.
template <bool ON>
struct MixBias {
  v4f* lds;
  __device__ __forceinline__ MixBias(const MixArgs& a, int64_t h0, int lane, v4f* lds_) : lds(lds_) {
    if (ON && lane < 12) {
      const int64_t col = lane < 8 ? h0 * 4 + 8 * lane : 4 * a.h + h0 * 2 + 8 * (lane - 8);
      lds[lane] = *reinterpret_cast<const v4f*>(static_cast<const uint16_t*>(a.abias) + col);
    }
  }
  __device__ __forceinline__ static v4f add8(v4f piece, v4f bias) {
    return narrow(widen_lo(piece) + widen_lo(bias), widen_hi(piece) + widen_hi(bias));
  }
  __device__ __forceinline__ void apply(MixRaw& x, int lane) const {
    if constexpr (!ON) return;
    const v4f bd = lds[lane & 7], bn = lds[8 + (lane & 3)];
    x.dl[0] = add8(x.dl[0], bd);
    x.dl[1] = add8(x.dl[1], bd);
    x.nz = add8(x.nz, bn);
  }
};

// Buffer descriptors of one batch row (range ends at token T) and row bytes.
struct MixRows {
  Rsrc q, k, v, dl, nz;
  uint32_t rq, rk, rv, rd, rn;       // row bytes
  uint32_t cq, ck, cv, cd, cn;       // byte offset of the wave's first head within a row
  __device__ __forceinline__ MixRows(const MixArgs& a, int64_t bb, int64_t h0) {
    const int64_t T = a.t;
    rq = static_cast<uint32_t>(a.ldq * 2);
    rk = static_cast<uint32_t>(a.ldk * 2);
    rv = static_cast<uint32_t>(a.ldv * 2);
    rd = static_cast<uint32_t>(a.ldd * 2);
    rn = static_cast<uint32_t>(a.ldn * 2);
    q = make_rsrc(as_f(a.q, bb * T * rq), static_cast<uint32_t>(T) * rq);
    k = make_rsrc(as_f(a.k, bb * T * rk), static_cast<uint32_t>(T) * rk);
    v = make_rsrc(as_f(a.v, bb * T * rv), static_cast<uint32_t>(T) * rv);
    dl = make_rsrc(as_f(a.dl, bb * T * rd), static_cast<uint32_t>(T) * rd);
    nz = make_rsrc(as_f(a.nz, bb * T * rn), static_cast<uint32_t>(T) * rn);
    cq = cd = ck = static_cast<uint32_t>(h0) * 8u;  // 4 bf16 per head
    cv = static_cast<uint32_t>(h0) * 16u;           // 8 bf16 per head
    cn = static_cast<uint32_t>(h0) * 4u;            // 2 bf16 per head
  }
  __device__ __forceinline__ void load(MixRaw& x, const MixMap& mm, int64_t t0) const {
#pragma unroll
    for (int I = 0; I < 2; ++I) {
      const uint32_t t = static_cast<uint32_t>(t0 + mm.kq_tok[I]);
      x.q[I] = ld128<kNtLoad>(q, t * rq + cq + mm.kq_col);
      x.k[I] = ld128<kNtLoad>(k, t * rk + ck + mm.kq_col);
      x.dl[I] = ld128<kNtLoad>(dl, t * rd + cd + mm.kq_col);
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const uint32_t t = static_cast<uint32_t>(t0 + mm.v_tok[I]);
      x.v[I] = ld128<kNtLoad>(v, t * rv + cv + mm.v_col);
    }
    const uint32_t t = static_cast<uint32_t>(t0 + mm.nz_tok);
    x.nz = ld128<false>(nz, t * rn + cn + mm.nz_col);
  }
};

// Transformed inputs of a tile into the LDS slot regions (K, Q, D, V, P, R of
// an FwdTile or BwdTile layout).
template <int K, int Q, int D, int V, int P, int R>
__device__ __forceinline__ void mix_put(const MixRaw& x, const MixMap& mm, float* tile) {
#pragma unroll
  for (int I = 0; I < 2; ++I) {
    *reinterpret_cast<v4f*>(&tile[K + mm.kq_lds[I][0]]) = unit_silu(widen_lo(x.k[I]));
    *reinterpret_cast<v4f*>(&tile[K + mm.kq_lds[I][1]]) = unit_silu(widen_hi(x.k[I]));
    *reinterpret_cast<v4f*>(&tile[Q + mm.kq_lds[I][0]]) = unit_silu(widen_lo(x.q[I]));
    *reinterpret_cast<v4f*>(&tile[Q + mm.kq_lds[I][1]]) = unit_silu(widen_hi(x.q[I]));
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const v4f z = e ? widen_hi(x.dl[I]) : widen_lo(x.dl[I]);
      v4f d;
#pragma unroll
      // The reference's exp(-softplus(z)) as written (train_6layer.py:690-698),
      // not the algebraically equal sigmoid(-z), which rounds differently.
      for (int i = 0; i < 4; ++i) d[i] = decay_(z[i]);
      *reinterpret_cast<v4f*>(&tile[D + mm.kq_lds[I][e]]) = d;
    }
  }
#pragma unroll
  for (int I = 0; I < 4; ++I) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const v4f z = e ? widen_hi(x.v[I]) : widen_lo(x.v[I]);
      v4f o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = silu_(z[i]);
      *reinterpret_cast<v4f*>(&tile[V + mm.v_lds[I][e]]) = o;
    }
  }
  const v4f lo = widen_lo(x.nz), hi = widen_hi(x.nz);  // (p, r) of heads 0, 1 | 2, 3
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float zp = e < 2 ? lo[2 * e] : hi[2 * e - 4];
    const float zr = e < 2 ? lo[2 * e + 1] : hi[2 * e - 3];
    tile[P + mm.nz_lds[e]] = softplus_(zp) + kNoiseFloor;
    tile[R + mm.nz_lds[e]] = softplus_(zr) + kNoiseFloor;
  }
}

// ------------------------------------------------------------ readout epilogue
// The mixer's readout (train_6layer.py:719-729) per head of 8 values:
//   out = RMSNorm(bf16(read)) * w * silu(gate),
// where RMSNorm computes in float32, eps defaulting to the float32 epsilon
// (torch's rms_norm with eps None).  Here the whole product is formed in
// float32 and rounded to bf16 once.  A head's 8 values sit in a lane pair
// (half = lane & 1 holds values 4 half .. + 3), so the squared norm and the
// backward's dot product are completed with one DPP exchange.

// Four bf16 values (a 64-bit piece) to float32, and float32 to a bf16 piece.
__device__ __forceinline__ v4f widen4(v2f piece) {
  const v2u w = __builtin_bit_cast(v2u, piece);
  v4f out;
  out[0] = __builtin_bit_cast(float, w[0] << 16);
  out[1] = __builtin_bit_cast(float, w[0] & 0xffff0000u);
  out[2] = __builtin_bit_cast(float, w[1] << 16);
  out[3] = __builtin_bit_cast(float, w[1] & 0xffff0000u);
  return out;
}
__device__ __forceinline__ v2f narrow4(v4f x) {
  v2u w;
  w[0] = narrow2(x[0], x[1]);
  w[1] = narrow2(x[2], x[3]);
  return __builtin_bit_cast(v2f, w);
}

// Buffer descriptors and lane offsets of the epilogue's [B, T, H * 8] streams
// (bf16 unless noted) for one batch row.
struct MixEpi {
  Rsrc gate, out, yb, gout, ggate;
  uint32_t rg, cg;    // gate row bytes; lane byte offset in a row
  uint32_t ro, co;    // contiguous bf16 rows (H * 16 bytes); lane byte offset
  uint32_t rgg;       // ggate row bytes (bf16 layout)
  float w[4], eps;
  bool precise;
  __device__ __forceinline__ MixEpi(const MixArgs& a, int64_t bb, int64_t h0, int lane, bool backward) {
    const int64_t T = a.t;
    const uint32_t yh = static_cast<uint32_t>((lane >> 1) & 15), half = static_cast<uint32_t>(lane & 1);
    precise = a.precise != 0;
    rg = static_cast<uint32_t>(a.ldg * 2);
    cg = (static_cast<uint32_t>(h0) + yh) * 16u + half * 8u;
    ro = static_cast<uint32_t>(a.h) * 16u;
    co = cg;
    rgg = static_cast<uint32_t>(a.ldgg ? a.ldgg : 8 * a.h) * 2u;
    const uint32_t tro = static_cast<uint32_t>(T) * ro, trw = precise ? 2u * tro : tro;
    const uint32_t trg = (precise ? 2u : 1u) * static_cast<uint32_t>(T) * rgg;
    gate = make_rsrc(as_f(a.gate, bb * T * rg), static_cast<uint32_t>(T) * rg);
    yb = make_rsrc(as_f(a.yb, bb * tro), tro);
    if (backward) {
      gout = make_rsrc(as_f(a.gout, bb * tro), tro);
      ggate = make_rsrc(as_f(a.ggate, bb * trg), trg);
      out = gout;
    } else {
      out = make_rsrc(as_f(a.out, bb * trw), trw);
      gout = ggate = out;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = a.norm_w[4 * half + i];
    eps = a.norm_eps;
  }
  // 1 / sqrt(mean of the head's 8 squares + eps), from this lane's four values.
  __device__ __forceinline__ float inv_rms(v4f x) const {
    float ss = x[0] * x[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) ss = fmaf(x[i], x[i], ss);
    ss += dpp<kXor1>(ss);
    return __builtin_amdgcn_rsqf(fmaf(ss, 0.125f, eps));
  }
  // Store a float32 result as bf16 (or float32 when precise) at byte offset
  // off of the bf16 layout.
  __device__ __forceinline__ void put4(Rsrc r, uint32_t off, v4f x) const {
    if (precise) st128<kNtStore>(r, x, 2u * off, 0);
    else st64(r, narrow4(x), off, 0);
  }
};

template <bool EPI, bool BIAS>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(1, 1))) void mixer_forward_kernel(MixArgs a) {
  __shared__ float tile[2 * FwdTile::SIZE];
  __shared__ float ckst[kRecFloats];
  const int lane = threadIdx.x;
  const int g = lane & 3, s = lane >> 2;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t bb = n0 / a.h, h0 = n0 - bb * a.h;
  const int64_t T = a.t;
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const uint32_t yrow = static_cast<uint32_t>(a.h) * 32u;
  const MixRows rows(a, bb, h0);
  const MixMap mm(lane, FwdTile::SIZE);
  __shared__ v4f bias_lds[BIAS ? 12 : 1];
  const MixBias<BIAS> bias(a, h0, lane, bias_lds);
  const Rsrc ry = make_rsrc(EPI ? a.m0 : a.y + bb * T * a.h * 8, EPI ? 0u : static_cast<uint32_t>(T) * yrow);
  const uint32_t ycol = static_cast<uint32_t>(h0) * 32u + mm.y_col;
  const MixEpi ep(a, bb, h0, lane, false);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 32, SPW * nbp * 128u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 16, SPW * nbp * 64u);
  const Rsrc rm0 = make_rsrc(a.m0 + n0 * 32, SPW * 128u);
  const Rsrc rc0 = make_rsrc(a.c0 + n0 * 16, SPW * 64u);
  const Rsrc rmT = make_rsrc(a.mT + n0 * 32, SPW * 128u);
  const Rsrc rcT = make_rsrc(a.cT + n0 * 16, SPW * 64u);

  const BelOff unit(s, g, 128u, 64u);
  FwdCore<false> core(lane, a.floor, a.chunk, nbp, ckst);
  load_bel(core.b, rm0, rc0, unit, 0, 0);
  core.store_ckpt(0, rbm, rbc);

  struct Out {
    v4f y[8];
  };
  auto take_y = [&](Out& o) __attribute__((always_inline)) {
#pragma unroll
    for (int I = 0; I < 8; ++I) o.y[I] = *reinterpret_cast<const v4f*>(&tile[FwdTile::V + mm.y_lds[I]]);
  };
  // Gate pieces of the tile whose readouts are stored next.
  v2f gt[8];
  auto load_gate = [&](int64_t t0) __attribute__((always_inline)) {
#pragma unroll
    for (int I = 0; I < 8; ++I)
      gt[I] = __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(
                                           ep.gate, static_cast<int>((t0 + mm.y_tok[I]) * ep.rg + ep.cg), 0, 0));
  };
  auto store_y = [&](const Out& o, int64_t t0) __attribute__((always_inline)) {
#pragma unroll
    for (int I = 0; I < 8; ++I) {
      const uint32_t t = static_cast<uint32_t>(t0 + mm.y_tok[I]);
      if constexpr (EPI) {
        const v2f yb = narrow4(o.y[I]);  // read.to(bf16)
        const v4f y = widen4(yb), z = widen4(gt[I]);
        const float r = ep.inv_rms(y);
        v4f x;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = y[i] * r * ep.w[i] * silu_(z[i]);
        ep.put4(ep.out, t * ep.ro + ep.co, x);
        st64(ep.yb, yb, t * ep.ro + ep.co, 0);
      } else {
        st128<kNtStore>(ry, o.y[I], t * yrow + ycol, 0);
      }
    }
  };

  // As the float32 forward: tile i + 1 loads while tile i computes; with the
  // epilogue, the gate of tile i loads then too (it is used when tile i's
  // readouts leave, during tile i + 1).
  const int64_t ntiles = (T + LT - 1) / LT;
  MixRaw st;
  rows.load(st, mm, 0);
  for (int64_t i = 0; i < ntiles; ++i) {
    Out yo;
    if (i > 0) take_y(yo);
    __builtin_amdgcn_sched_barrier(0);
    bias.apply(st, lane);
    mix_put<FwdTile::K, FwdTile::Q, FwdTile::D, FwdTile::V, FwdTile::P, FwdTile::R>(st, mm, tile);
    __builtin_amdgcn_sched_barrier(0);
    if (i > 0) store_y(yo, (i - 1) * LT);
    if (i + 1 < ntiles) rows.load(st, mm, (i + 1) * LT);
    if constexpr (EPI) load_gate(i * LT);
    __builtin_amdgcn_sched_barrier(0);
    const int64_t t0 = i * LT;
    core.run_sub(tile, t0, T, rbm, rbc);
    if (t0 + TT < T) core.run_sub(tile + FwdTile::SIZE, t0 + TT, T, rbm, rbc);
  }
  {
    Out yo;
    take_y(yo);
    store_y(yo, (ntiles - 1) * LT);
  }
  store_bel(core.b, rmT, rcT, unit, 0, 0);
  core.store_ckpt(static_cast<uint32_t>(a.nb), rbm, rbc);
}

// Gradient outputs: contiguous [B, T, H * w] rows, bfloat16 or float32.
struct MixGrads {
  Rsrc q, k, v, dl, nz;
  uint32_t rq, rk, rv, rd, rn;  // row bytes of the bf16 layout
  uint32_t ckq, cv, cn;         // byte offset of the wave's first head, bf16 layout
  bool f32;
  __device__ __forceinline__ MixGrads(const MixArgs& a, int64_t bb, int64_t h0) {
    const int64_t T = a.t, H = a.h;
    f32 = a.grad_f32 != 0;
    // Row strides: the caller's, or contiguous rows of 4 / 8 / 2 values per head.
    rq = static_cast<uint32_t>(a.ldgq ? a.ldgq : 4 * H) * 2u;
    rk = static_cast<uint32_t>(a.ldgk ? a.ldgk : 4 * H) * 2u;
    rv = static_cast<uint32_t>(a.ldgv ? a.ldgv : 8 * H) * 2u;
    rd = static_cast<uint32_t>(a.ldgd ? a.ldgd : 4 * H) * 2u;
    rn = static_cast<uint32_t>(a.ldgn ? a.ldgn : 2 * H) * 2u;
    ckq = static_cast<uint32_t>(h0) * 8u;
    cv = static_cast<uint32_t>(h0) * 16u;
    cn = static_cast<uint32_t>(h0) * 4u;
    // Offsets are computed in the bf16 layout; float32 rows are twice as long.
    const int64_t e = f32 ? 2 : 1;
    const uint32_t tq = static_cast<uint32_t>(T * e) * rq, tk = static_cast<uint32_t>(T * e) * rk,
                   tv = static_cast<uint32_t>(T * e) * rv, td = static_cast<uint32_t>(T * e) * rd,
                   tn = static_cast<uint32_t>(T * e) * rn;
    q = make_rsrc(as_f(a.gq, bb * tq), tq);
    k = make_rsrc(as_f(a.gk, bb * tk), tk);
    v = make_rsrc(as_f(a.gv, bb * tv), tv);
    const bool dyn = a.gdl != nullptr;
    dl = make_rsrc(as_f(dyn ? a.gdl : a.gq, dyn ? bb * td : 0), dyn ? td : 0u);
    nz = make_rsrc(as_f(dyn ? a.gnz : a.gq, dyn ? bb * tn : 0), dyn ? tn : 0u);
  }
  // One piece of 8 values (lo = first four, hi = last four) at the bf16
  // byte offset `off`: bf16 as one 16-byte piece, float32 as two.
  __device__ __forceinline__ void put8(Rsrc r, uint32_t off, v4f lo, v4f hi) const {
    if (f32) {
      st128<kNtStore>(r, lo, 2u * off, 0);
      st128<kNtStore>(r, hi, 2u * off + 16u, 0);
    } else {
      st128<kNtStore>(r, narrow(lo, hi), off, 0);
    }
  }
};

template <bool DYN, bool EPI, bool BIAS>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(1, 1))) void mixer_backward_kernel(
    MixArgs a) {
  __shared__ float tile[2 * BwdTile::SIZE];
  const int lane = threadIdx.x;
  const int g = lane & 3, s = lane >> 2;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t bb = n0 / a.h, h0 = n0 - bb * a.h;
  const int64_t T = a.t;
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const uint32_t yrow = static_cast<uint32_t>(a.h) * 32u;
  const MixRows rows(a, bb, h0);
  const MixGrads gr(a, bb, h0);
  const MixMap mm(lane, BwdTile::SIZE);
  __shared__ v4f bias_lds[BIAS ? 12 : 1];
  const MixBias<BIAS> bias(a, h0, lane, bias_lds);
  const Rsrc rgy = make_rsrc(EPI ? a.m0 : a.gy + bb * T * a.h * 8, EPI ? 0u : static_cast<uint32_t>(T) * yrow);
  const uint32_t ycol = static_cast<uint32_t>(h0) * 32u + mm.y_col;
  const MixEpi ep(a, bb, h0, lane, true);
  // This lane's share of the norm-weight gradient, summed in LDS (a
  // loop-carried register set would push the kernel past the register file).
  __shared__ v4f dwl[EPI ? kWave : 1];
  if constexpr (EPI) dwl[lane] = v4f{0.f, 0.f, 0.f, 0.f};
  const Rsrc rbm = make_rsrc(a.bmr + n0 * nbp * 32, SPW * nbp * 128u);
  const Rsrc rbc = make_rsrc(a.bcr + n0 * nbp * 16, SPW * nbp * 64u);
  const RecOff ckoff(lane, nbp * 128u, nbp * 64u);

  const BelOff unit(s, g, 128u, 64u);
  BwdCore<false, DYN> core(s, g, a.floor);
  core.init(a.gmf, a.gcf, a.m0, n0, SPW, unit, s);
  const int64_t nb = a.nb;
  const int64_t ntiles = (nb + 1) / 2;

  struct Stage {
    MixRaw raw;
    v4f gy[8];  // without the epilogue
  };
  // Epilogue pieces of one sub-tile h (readout map instructions 4h .. 4h + 3).
  struct EpiHalf {
    v2f go[4], yb[4], gt[4];
  };
  auto load_raw = [&](Stage& x, int64_t J) __attribute__((always_inline)) { rows.load(x.raw, mm, J * 2 * SUB); };
  auto load_y = [&](Stage& x, int64_t J) __attribute__((always_inline)) {
    const int64_t t0 = J * 2 * SUB;
#pragma unroll
    for (int I = 0; I < 8; ++I)
      x.gy[I] = ld128<kNtLoad>(rgy, static_cast<uint32_t>(t0 + mm.y_tok[I]) * yrow + ycol);
  };
  auto load_epi = [&](EpiHalf& x, int64_t J, int h) __attribute__((always_inline)) {
    const int64_t t0 = J * 2 * SUB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t t = static_cast<uint32_t>(t0 + mm.y_tok[4 * h + i]);
      x.go[i] = ld64(ep.gout, t * ep.ro + ep.co, 0);
      x.yb[i] = ld64(ep.yb, t * ep.ro + ep.co, 0);
      x.gt[i] = ld64(ep.gate, t * ep.rg + ep.cg, 0);
    }
  };
  // The aux bias goes into the raw pieces here, so the pieces kept for the
  // chain rule hold the biased logits too.
  auto put = [&](Stage& x, int64_t J) __attribute__((always_inline)) {
    bias.apply(x.raw, lane);
    mix_put<BwdTile::K, BwdTile::Q, BwdTile::D, BwdTile::V, BwdTile::P, BwdTile::R>(x.raw, mm, tile);
    if constexpr (!EPI) {
#pragma unroll
      for (int I = 0; I < 8; ++I) *reinterpret_cast<v4f*>(&tile[BwdTile::GY + mm.y_lds[I]]) = x.gy[I];
    }
  };
  // The readout gradient gy of sub-tile h of tile J into LDS, per head
  // (n = y r, h = n w, out = h silu(z)):
  //   dL/dh = gout silu(z),  dL/dz = gout h silu'(z),  dL/dw += dL/dh n,
  //   gy = r (dL/dn - n mean(dL/dn n)) with dL/dn = dL/dh w.
  auto put_epi = [&](const EpiHalf& x, int64_t J, int h) __attribute__((always_inline)) {
    v4f dw = dwl[lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int I = 4 * h + i;
      const v4f y = widen4(x.yb[i]), z = widen4(x.gt[i]), go = widen4(x.go[i]);
      const float r = ep.inv_rms(y);
      v4f gz, gn, n;
      float dot = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float sg = sigmoid_(z[c]), sz = z[c] * sg;  // silu(z)
        const float dsz = fmaf(sz, -sg, sg + sz);         // silu'(z) = sg + silu(z) (1 - sg)
        n[c] = y[c] * r;
        const float gh = go[c] * sz;
        gz[c] = go[c] * (n[c] * ep.w[c]) * dsz;
        gn[c] = gh * ep.w[c];
        dw[c] = fmaf(gh, n[c], dw[c]);
        dot = fmaf(gn[c], n[c], dot);
      }
      dot += dpp<kXor1>(dot);
      v4f gy;
#pragma unroll
      for (int c = 0; c < 4; ++c) gy[c] = r * fmaf(-n[c], dot * 0.125f, gn[c]);
      *reinterpret_cast<v4f*>(&tile[BwdTile::GY + mm.y_lds[I]]) = gy;
      const uint32_t t = static_cast<uint32_t>(J * 2 * SUB + mm.y_tok[I]);
      ep.put4(ep.ggate, t * ep.rgg + ep.co, gz);
    }
    dwl[lane] = dw;
  };
  auto issue_ck = [&](float* tl, int64_t c) __attribute__((always_inline)) {
    lds_wait();
    const uint32_t cm = static_cast<uint32_t>(c) * 128u, cc = static_cast<uint32_t>(c) * 64u;
    dma16<kNtCkpt>(rbm, (tl + BwdTile::CK), ckoff.m0 + cm);
    dma16<kNtCkpt>(rbm, (tl + BwdTile::CK) + 256, ckoff.m1 + cm);
    dma16(rbc, (tl + BwdTile::CK) + 512, ckoff.c + cc);
  };
  // Projection gradients of tile J: the reverse left dL/d(transformed input)
  // in the LDS regions; the raw pieces of the tile give the chain rule.  The
  // pieces of tokens 8..15 (q, k, decay I = 1; v I = 2, 3) are written once
  // chunk 2J + 1 is reversed (HI), the rest and the noise once chunk 2J is
  // (LO), so half of the kept pieces are free during chunk 2J.
  auto write_grads = [&](const MixRaw& x, int64_t J, bool hi) __attribute__((always_inline)) {
    const int64_t t0 = J * 2 * SUB;
#pragma unroll
    for (int I = hi ? 1 : 0; I < (hi ? 2 : 1); ++I) {
      const uint32_t t = static_cast<uint32_t>(t0 + mm.kq_tok[I]);
      const int o0 = mm.kq_lds[I][0], o1 = mm.kq_lds[I][1];
      const v4f gk0 = *reinterpret_cast<const v4f*>(&tile[BwdTile::K + o0]);
      const v4f gk1 = *reinterpret_cast<const v4f*>(&tile[BwdTile::K + o1]);
      gr.put8(gr.k, t * gr.rk + gr.ckq + mm.kq_col, unit_silu_grad(widen_lo(x.k[I]), gk0),
              unit_silu_grad(widen_hi(x.k[I]), gk1));
      const v4f gq0 = *reinterpret_cast<const v4f*>(&tile[BwdTile::Q + o0]);
      const v4f gq1 = *reinterpret_cast<const v4f*>(&tile[BwdTile::Q + o1]);
      gr.put8(gr.q, t * gr.rq + gr.ckq + mm.kq_col, unit_silu_grad(widen_lo(x.q[I]), gq0),
              unit_silu_grad(widen_hi(x.q[I]), gq1));
      if constexpr (DYN) {
        v4f out[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const v4f z = e ? widen_hi(x.dl[I]) : widen_lo(x.dl[I]);
          const v4f gd = *reinterpret_cast<const v4f*>(&tile[BwdTile::D + (e ? o1 : o0)]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // d/dz exp(-softplus(z)) = -exp(-softplus(z)) sigmoid(z)
            // = -sigmoid(-z) sigmoid(z) = -sigmoid(|z|)^2 e^-|z| (the same
            // product whatever the sign of z), from one exponential and one
            // reciprocal.
            const float ea = exp_(-fabsf(z[i])), sa = rcp_(1.f + ea);
            out[e][i] = -gd[i] * (ea * sa) * sa;
          }
        }
        gr.put8(gr.dl, t * gr.rd + gr.ckq + mm.kq_col, out[0], out[1]);
      }
    }
#pragma unroll
    for (int I = hi ? 2 : 0; I < (hi ? 4 : 2); ++I) {
      const uint32_t t = static_cast<uint32_t>(t0 + mm.v_tok[I]);
      v4f out[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const v4f z = e ? widen_hi(x.v[I]) : widen_lo(x.v[I]);
        const v4f gv = *reinterpret_cast<const v4f*>(&tile[BwdTile::V + mm.v_lds[I][e]]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float sg = sigmoid_(z[i]);
          out[e][i] = gv[i] * sg * fmaf(z[i], 1.f - sg, 1.f);
        }
      }
      gr.put8(gr.v, t * gr.rv + gr.cv + mm.v_col, out[0], out[1]);
    }
    if (DYN && !hi) {
      const uint32_t t = static_cast<uint32_t>(t0 + mm.nz_tok);
      const v4f lo = widen_lo(x.nz), hi = widen_hi(x.nz);
      v4f out[2];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float zp = e < 2 ? lo[2 * e] : hi[2 * e - 4];
        const float zr = e < 2 ? lo[2 * e + 1] : hi[2 * e - 3];
        const float gp = tile[BwdTile::P + mm.nz_lds[e]] * sigmoid_(zp);
        const float grr = tile[BwdTile::R + mm.nz_lds[e]] * sigmoid_(zr);
        out[e >> 1][2 * (e & 1)] = gp;
        out[e >> 1][2 * (e & 1) + 1] = grr;
      }
      gr.put8(gr.nz, t * gr.rn + gr.cn + mm.nz_col, out[0], out[1]);
    }
  };
  auto chunk_len = [&](int64_t c) __attribute__((always_inline)) {
    return static_cast<int>((T - c * SUB) < SUB ? (T - c * SUB) : SUB);
  };
  auto run_chunk = [&](float* tl, int64_t c) __attribute__((always_inline)) {
    Bel b;
    bel_from_lds(b, tl + BwdTile::CK, s, g);
    if (c >= 2) issue_ck(tl, c - 2);
    core.run(tl, b, chunk_len(c));
  };

  // As the bf16-input backward: tile J's loads were issued during tile J + 1;
  // the raw pieces of the tile being written out are kept until its
  // gradients have left.
  // Tiles run from the last to the first; tile J's projection pieces were
  // loaded during tile J + 1 and are kept until its gradients have left.
  // Without the epilogue, tile J's gy is staged with them.  With it, the
  // epilogue pieces of one sub-tile at a time are staged: those of sub-tile
  // 1 (tokens 8..15, chunk 2J + 1) load during chunk 2J + 2 and form gy at the
  // tile's put; those of sub-tile 0 load at the put and form gy between the
  // two chunks.
  Stage st;
  MixRaw kept;
  EpiHalf eh;
  load_raw(st, ntiles - 1);
  if constexpr (EPI) load_epi(eh, ntiles - 1, 1);
  else load_y(st, ntiles - 1);
  issue_ck(tile, 2 * (ntiles - 1));
  if (2 * ntiles - 1 < nb) issue_ck(tile + BwdTile::SIZE, 2 * ntiles - 1);
  else if (ntiles > 1) issue_ck(tile + BwdTile::SIZE, 2 * ntiles - 3);
  for (int64_t J = ntiles - 1; J >= 0; --J) {
    vm_wait<0>();
    if (J + 1 < ntiles) {
      write_grads(kept, J + 1, false);
      write_grads(kept, J + 1, true);
    }
    __builtin_amdgcn_sched_barrier(0);
    lds_wait();
    put(st, J);
    if constexpr (EPI) put_epi(eh, J, 1);
    kept = st.raw;
    __builtin_amdgcn_sched_barrier(0);
    if (J > 0) {
      load_raw(st, J - 1);
      if constexpr (!EPI) load_y(st, J - 1);
    }
    if constexpr (EPI) load_epi(eh, J, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (2 * J + 1 < nb) run_chunk(tile + BwdTile::SIZE, 2 * J + 1);
    if constexpr (EPI) {
      __builtin_amdgcn_sched_barrier(0);
      put_epi(eh, J, 0);
      if (J > 0) load_epi(eh, J - 1, 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    run_chunk(tile, 2 * J);
  }
  write_grads(kept, 0, false);
  write_grads(kept, 0, true);
  core.store_initial(a.gm0, a.gc0, n0, SPW, unit);
  if constexpr (EPI) {
    // Sum the weight-gradient shares of the 32 lanes of each half; lanes 0
    // and 1 write the wave's 8 partials.
    v4f dw = dwl[lane];
#pragma unroll
    for (int m = 2; m < kWave; m *= 2)
#pragma unroll
      for (int i = 0; i < 4; ++i) dw[i] += __shfl_xor(dw[i], m);
    if (lane < 2) *reinterpret_cast<v4f*>(a.gw_part + static_cast<int64_t>(blockIdx.x) * 8 + lane * 4) = dw;
  }
}

}  // namespace
}  // namespace r4

hipError_t launch_mixer_forward(const MixArgs& a, hipStream_t stream) {
  const int64_t blocks = a.b * a.h / r4::SPW;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  // The aux bias only comes with the readout epilogue (the block entry points).
  if (a.gate != nullptr && a.abias != nullptr)
    hipLaunchKernelGGL((r4::mixer_forward_kernel<true, true>), grid, block, 0, stream, a);
  else if (a.gate != nullptr) hipLaunchKernelGGL((r4::mixer_forward_kernel<true, false>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((r4::mixer_forward_kernel<false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_mixer_backward(const MixArgs& a, hipStream_t stream) {
  const int64_t blocks = a.b * a.h / r4::SPW;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  const bool dyn = a.gdl != nullptr, epi = a.gate != nullptr;
  if (dyn && epi && a.abias != nullptr)
    hipLaunchKernelGGL((r4::mixer_backward_kernel<true, true, true>), grid, block, 0, stream, a);
  else if (dyn && epi) hipLaunchKernelGGL((r4::mixer_backward_kernel<true, true, false>), grid, block, 0, stream, a);
  else if (dyn) hipLaunchKernelGGL((r4::mixer_backward_kernel<true, false, false>), grid, block, 0, stream, a);
  else if (epi) hipLaunchKernelGGL((r4::mixer_backward_kernel<false, true, false>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((r4::mixer_backward_kernel<false, false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace bssm
