// gfx950 kernels for D = 4, M = 8 (bayes_ssm/persistent_bayes_chunked_d4m8.cu
// is the reference extension for this shape): the float32 and bf16-input
// forward and backward, on the rotated per-lane layout and LDS tiles of
// bssm_rot4.h.

#include "bssm_rot4.h"

namespace bssm {
namespace r4 {

// F: format of keys, queries and values (InFmt): float32, bfloat16 or float8.
template <bool FIXED, int F>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(1, 1))) void forward_kernel(FwdArgs a) {
  constexpr bool H = F == kInBf16, Q8 = F >= kInE4M3, W = F == kInF32;
  __shared__ float tile[2 * FwdTile::SIZE];
  __shared__ float ckst[kRecFloats];  // checkpoint staging
  const int lane = threadIdx.x;
  const int g = lane & 3, s = lane >> 2;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t T = a.t;
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  const uint32_t row4 = static_cast<uint32_t>(T) * 16u, row8 = static_cast<uint32_t>(T) * 32u,
                 row1 = static_cast<uint32_t>(T) * 4u;
  // Keys, queries and values take half (bf16) or a quarter (float8) of the float32 row bytes.
  const uint32_t kb = H ? 2u : Q8 ? 4u : 1u;
  const Rsrc rk = make_rsrc(byte_offset(a.k, n0 * T * 16 / kb), valid * row4 / kb);
  const Rsrc rq = make_rsrc(byte_offset(a.q, n0 * T * 16 / kb), valid * row4 / kb);
  const Rsrc rv = make_rsrc(byte_offset(a.v, n0 * T * 32 / kb), valid * row8 / kb);
  const Rsrc ry = make_rsrc(a.y + n0 * T * 8, valid * row8);
  const Rsrc rd = make_rsrc(FIXED ? a.y : a.d + n0 * T * 4, valid * row4);
  const Rsrc rp = make_rsrc(FIXED ? a.y : a.p + n0 * T, valid * row1);
  const Rsrc rr = make_rsrc(FIXED ? a.y : a.r + n0 * T, valid * row1);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 32, valid * nbp * 128u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 16, valid * nbp * 64u);
  const Rsrc rm0 = make_rsrc(a.m0 + n0 * 32, valid * 128u);
  const Rsrc rc0 = make_rsrc(a.c0 + n0 * 16, valid * 64u);
  const Rsrc rmT = make_rsrc(a.mT + n0 * 32, valid * 128u);
  const Rsrc rcT = make_rsrc(a.cT + n0 * 16, valid * 64u);

  const Map mp(lane, row4, row8, row1);
  const HalfMap hm(lane, FwdTile::SIZE, row4 / 2, row8 / 2);
  const QuarterMap qm(lane, FwdTile::SIZE, row4 / 4, row8 / 4);
  const uint32_t off1 = static_cast<uint32_t>(lane >> 2) * row1 + static_cast<uint32_t>(lane & 3) * 16u;
  const int dst1 = ((lane & 3) >> 1) * FwdTile::SIZE + 4 * (2 * (lane >> 2) + (lane & 1));

  const BelOff unit(s, g, 128u, 64u);
  FwdCore<FIXED> core(lane, a.floor, a.chunk, nbp, ckst);
  load_bel(core.b, rm0, rc0, unit, 0, 0);
  core.store_ckpt(0, rbm, rbc);

  using Stage = std::conditional_t<H, FwdStageH, std::conditional_t<Q8, FwdStageQ, FwdStage>>;
  auto load = [&](Stage& x, int64_t t0) __attribute__((always_inline)) {
    if constexpr (Q8) {
      // A float8 key or query row of 16 tokens is half a 128-byte line: the
      // cached hint keeps the other half in L2 for the next tile (the
      // nontemporal one refetched it, about 6 B per token more traffic).
      const uint32_t sk = static_cast<uint32_t>(t0) * 4u, sv = static_cast<uint32_t>(t0) * 8u;
      x.k = ld128<false>(rk, qm.k_off + sk);
      x.q = ld128<false>(rq, qm.k_off + sk);
#pragma unroll
      for (int I = 0; I < 2; ++I) x.v[I] = ld128<kNtLoad>(rv, qm.v_off[I] + sv);
    }
    if constexpr (H) {
      const uint32_t sk = static_cast<uint32_t>(t0) * 8u, sv = static_cast<uint32_t>(t0) * 16u;
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        x.k[I] = ld128<kNtLoad>(rk, hm.k_off[I] + sk);
        x.q[I] = ld128<kNtLoad>(rq, hm.k_off[I] + sk);
      }
#pragma unroll
      for (int I = 0; I < 4; ++I) x.v[I] = ld128<kNtLoad>(rv, hm.v_off[I] + sv);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t s4 = static_cast<uint32_t>(t0 + TT * h) * 16u, s8 = static_cast<uint32_t>(t0 + TT * h) * 32u;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (W) {
          x.k[2 * h + j] = ld128<kNtLoad>(rk, mp.d4[j] + s4);
          x.q[2 * h + j] = ld128<kNtLoad>(rq, mp.d4[j] + s4);
        }
        if constexpr (!FIXED) x.d[2 * h + j] = ld128<kNtLoad>(rd, mp.d4[j] + s4);
      }
      if constexpr (W) {
#pragma unroll
        for (int j = 0; j < 4; ++j) x.v[4 * h + j] = ld128<kNtLoad>(rv, mp.d8[j] + s8);
      }
    }
    if constexpr (!FIXED) {
      const uint32_t s1 = static_cast<uint32_t>(t0) * 4u;
      x.p = ld128<false>(rp, off1 + s1);
      x.r = ld128<false>(rr, off1 + s1);
    }
  };
  auto put = [&](const Stage& x) __attribute__((always_inline)) {
    if constexpr (Q8) {
      const v4u wk = __builtin_bit_cast(v4u, x.k), wq = __builtin_bit_cast(v4u, x.q);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        *reinterpret_cast<v4f*>(&tile[FwdTile::K + qm.k_lds[u]]) = widen_f8<F>(wk[u]);
        *reinterpret_cast<v4f*>(&tile[FwdTile::Q + qm.k_lds[u]]) = widen_f8<F>(wq[u]);
      }
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        const v4u wv = __builtin_bit_cast(v4u, x.v[I]);
#pragma unroll
        for (int w = 0; w < 4; ++w) *reinterpret_cast<v4f*>(&tile[FwdTile::V + qm.v_lds[I][w]]) = widen_f8<F>(wv[w]);
      }
    }
    if constexpr (H) {
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        *reinterpret_cast<v4f*>(&tile[FwdTile::K + hm.k_lds[I][0]]) = widen_lo(x.k[I]);
        *reinterpret_cast<v4f*>(&tile[FwdTile::K + hm.k_lds[I][1]]) = widen_hi(x.k[I]);
        *reinterpret_cast<v4f*>(&tile[FwdTile::Q + hm.k_lds[I][0]]) = widen_lo(x.q[I]);
        *reinterpret_cast<v4f*>(&tile[FwdTile::Q + hm.k_lds[I][1]]) = widen_hi(x.q[I]);
      }
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        *reinterpret_cast<v4f*>(&tile[FwdTile::V + hm.v_lds[I][0]]) = widen_lo(x.v[I]);
        *reinterpret_cast<v4f*>(&tile[FwdTile::V + hm.v_lds[I][1]]) = widen_hi(x.v[I]);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float* tl = tile + h * FwdTile::SIZE;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (W) {
          *reinterpret_cast<v4f*>(&(tl + FwdTile::K)[256 * j + 4 * lane]) = x.k[2 * h + j];
          *reinterpret_cast<v4f*>(&(tl + FwdTile::Q)[256 * j + 4 * lane]) = x.q[2 * h + j];
        }
        if constexpr (!FIXED) *reinterpret_cast<v4f*>(&(tl + FwdTile::D)[256 * j + 4 * lane]) = x.d[2 * h + j];
      }
      if constexpr (W) {
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<v4f*>(&(tl + FwdTile::V)[256 * j + 4 * lane]) = x.v[4 * h + j];
      }
    }
    if constexpr (!FIXED) {
      *reinterpret_cast<v4f*>(&(tile + FwdTile::P)[dst1]) = x.p;
      *reinterpret_cast<v4f*>(&(tile + FwdTile::R)[dst1]) = x.r;
    }
  };

  // Readouts of a tile: read out of LDS before the next tile is written
  // there, stored after that tile's loads have been awaited.
  struct FwdOut {
    v4f y[8];
  };
  auto take_y = [&](FwdOut& o) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o.y[4 * h + j] = *reinterpret_cast<const v4f*>(&(tile + h * FwdTile::SIZE + FwdTile::V)[256 * j + 4 * lane]);
  };
  auto store_y = [&](const FwdOut& o, int64_t t0) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t th = t0 + TT * h;
      const int len = static_cast<int>((T - th) < TT ? (T - th) : TT);
      const uint32_t s8 = static_cast<uint32_t>(th) * 32u;
#pragma unroll
      for (int j = 0; j < 4; ++j) st128<kNtStore>(ry, o.y[4 * h + j], mp.t8[j] < len ? mp.d8[j] : kOob, s8);
    }
  };

  // Tile i: its loads were issued at the start of tile i - 1 (the compiler
  // waits for them before they are written to LDS); the readouts of tile
  // i - 1 leave LDS first and are stored after that wait, then the loads of
  // tile i + 1 are issued and the two sub-tiles computed.
  const int64_t ntiles = (T + LT - 1) / LT;
  Stage st;
  load(st, 0);
  for (int64_t i = 0; i < ntiles; ++i) {
    FwdOut yo;
    if (i > 0) take_y(yo);
    __builtin_amdgcn_sched_barrier(0);
    put(st);
    __builtin_amdgcn_sched_barrier(0);
    if (i > 0) store_y(yo, (i - 1) * LT);
    if (i + 1 < ntiles) load(st, (i + 1) * LT);
    __builtin_amdgcn_sched_barrier(0);
    const int64_t t0 = i * LT;
    core.run_sub(tile, t0, T, rbm, rbc);
    if (t0 + TT < T) core.run_sub(tile + FwdTile::SIZE, t0 + TT, T, rbm, rbc);
  }
  {
    FwdOut yo;
    take_y(yo);
    store_y(yo, (ntiles - 1) * LT);
  }
  store_bel(core.b, rmT, rcT, unit, 0, 0);
  core.store_ckpt(static_cast<uint32_t>(a.nb), rbm, rbc);
}

// ------------------------------------------- register-staged tile backward
// A 16-token tile (chunks 2J, 2J + 1) is staged in registers while the
// previous tile is replayed and reversed from LDS; at the tile boundary the
// gradients of the finished tile leave LDS for registers, the staged inputs
// take their place, and the gradients are stored.  Float32 streams (all of
// them for F = float32; d and gy otherwise) move as whole 16-token row
// segments per instruction (TileMap).  With bfloat16 or float8 keys, values
// and queries those three arrive in their format and are widened into the
// same float32 slot layout, and their gradients are narrowed on the way out
// (bf16: round to nearest even; float8: torch's rounding).  Checkpoint
// records arrive by LDS-DMA into their chunk's slot once its chunk has read
// its own.
//
// bf16 piece maps (16-byte pieces, 16-token tile starting at t0):
//   k, q: row 8I + (l & 7), tokens t0 + 2 (l >> 3) and + 1 (I < 2)
//   v:    row 4I + (l & 3), token t0 + (l >> 2) (I < 4)
struct BwdStageF {
  v4f k[4], q[4], v[8], d[4], gy[8], p, r;
};
struct BwdOutF {
  v4f k[4], q[4], v[8], d[4], p, r;
};
struct BwdStageH {
  v4f k[2], q[2], v[4], d[4], gy[8], p, r;
};
struct BwdOutH {
  v4f k[2], q[2], v[4], d[4], p, r;
};
// The same with float8 keys, queries and values (QuarterMap pieces).
struct BwdStageQ {
  v4f k, q, v[2], d[4], gy[8], p, r;
};
struct BwdOutQ {
  v4f k, q, v[2], d[4], p, r;
};

// F: format of keys, values, queries and their gradients (InFmt).  IV:
// checkpoint interval, 8 (a record per chunk slot) or 16 (a record per tile:
// the tile's second chunk starts from the belief advanced over its first).
template <bool FIXED, bool DYN, int F, int IV>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(1, 1))) void backward_tile_kernel(
    BwdArgs a) {
  static_assert(IV == SUB || IV == 2 * SUB, "checkpoint interval of one or two chunk slots");
  constexpr bool Q8 = F >= kInE4M3, W = F == kInF32;
  constexpr uint32_t kb = Q8 ? 4u : W ? 1u : 2u;  // float32 row bytes per stream row byte
  __shared__ float tile[2 * BwdTile::SIZE];
  const int lane = threadIdx.x;
  const int g = lane & 3, s = lane >> 2;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * SPW;
  const int64_t T = a.t;
  const uint32_t valid = static_cast<uint32_t>((a.n - n0) < SPW ? (a.n - n0) : SPW);
  const uint32_t row4 = static_cast<uint32_t>(T) * 16u, row8 = static_cast<uint32_t>(T) * 32u,
                 row1 = static_cast<uint32_t>(T) * 4u;
  const uint32_t row4h = row4 / kb, row8h = row8 / kb;
  const int64_t e4 = 16 / kb, e8 = 32 / kb;  // stream bytes per token of k / v
  const Rsrc rk = make_rsrc(byte_offset(a.k, n0 * T * e4), valid * row4h);
  const Rsrc rq = make_rsrc(byte_offset(a.q, n0 * T * e4), valid * row4h);
  const Rsrc rv = make_rsrc(byte_offset(a.v, n0 * T * e8), valid * row8h);
  const Rsrc rgk = make_rsrc(byte_offset(a.gk, n0 * T * e4), valid * row4h);
  const Rsrc rgq = make_rsrc(byte_offset(a.gq, n0 * T * e4), valid * row4h);
  const Rsrc rgv = make_rsrc(byte_offset(a.gv, n0 * T * e8), valid * row8h);
  const Rsrc rgy = make_rsrc(a.gy + n0 * T * 8, valid * row8);
  const Rsrc rd = make_rsrc(FIXED ? a.gy : a.d + n0 * T * 4, valid * row4);
  const Rsrc rp = make_rsrc(FIXED ? a.gy : a.p + n0 * T, valid * row1);
  const Rsrc rr = make_rsrc(FIXED ? a.gy : a.r + n0 * T, valid * row1);
  const Rsrc rgd = make_rsrc(a.gd ? a.gd + n0 * T * 4 : a.gy, a.gd ? valid * row4 : 0u);
  const Rsrc rgp = make_rsrc(a.gp ? a.gp + n0 * T : a.gy, a.gp ? valid * row1 : 0u);
  const Rsrc rgr = make_rsrc(a.gr ? a.gr + n0 * T : a.gy, a.gr ? valid * row1 : 0u);
  const uint32_t nbp = static_cast<uint32_t>(a.nb + 1);
  const Rsrc rbm = make_rsrc(a.bm + n0 * nbp * 32, valid * nbp * 128u);
  const Rsrc rbc = make_rsrc(a.bc + n0 * nbp * 16, valid * nbp * 64u);

  const TileMap tm(lane, row4, row8, row1);
  const HalfMap hm(lane, BwdTile::SIZE, row4h, row8h);
  const QuarterMap qm(lane, BwdTile::SIZE, row4h, row8h);

  const BelOff unit(s, g, 128u, 64u);
  BwdCore<FIXED, DYN> core(s, g, a.floor);
  core.init(a.gmf, a.gcf, a.m0, n0, valid, unit, s);
  const RecOff ckoff(lane, nbp * 128u, nbp * 64u);
  const int64_t nb = a.nb;                    // checkpoint chunks of IV tokens
  const int64_t nsub = (T + SUB - 1) / SUB;   // chunk slots of SUB tokens
  const int64_t ntiles = (nsub + 1) / 2;

  using Stage = std::conditional_t<W, BwdStageF, std::conditional_t<Q8, BwdStageQ, BwdStageH>>;
  using Out = std::conditional_t<W, BwdOutF, std::conditional_t<Q8, BwdOutQ, BwdOutH>>;
  auto load = [&](Stage& x, int64_t J) __attribute__((always_inline)) {
    const int64_t t0 = J * 2 * SUB;
    const uint32_t sk = static_cast<uint32_t>(t0 * e4), sv = static_cast<uint32_t>(t0 * e8);
    const uint32_t s4 = static_cast<uint32_t>(t0) * 16u, s8 = static_cast<uint32_t>(t0) * 32u;
    // Pieces of tokens at or past T (a partial last tile) are not requested.
    const bool full = t0 + 2 * SUB <= T;
    const bool in4 = full || t0 + tm.t4 < T, in8 = full || t0 + tm.t8 < T, in1 = full || t0 + tm.t1 < T;
    if constexpr (W) {
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        x.k[I] = ld128<kNtLoad>(rk, in4 ? tm.o4[I] : kOob, s4);
        x.q[I] = ld128<kNtLoad>(rq, in4 ? tm.o4[I] : kOob, s4);
      }
#pragma unroll
      for (int I = 0; I < 8; ++I) x.v[I] = ld128<kNtLoad>(rv, in8 ? tm.o8[I] : kOob, s8);
    } else if constexpr (Q8) {
      // Half-line float8 rows: cached, as in the forward.
      x.k = ld128<false>(rk, qm.k_off + sk);
      x.q = ld128<false>(rq, qm.k_off + sk);
#pragma unroll
      for (int I = 0; I < 2; ++I) x.v[I] = ld128<kNtLoad>(rv, qm.v_off[I] + sv);
    } else {
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        x.k[I] = ld128<kNtLoad>(rk, hm.k_off[I] + sk);
        x.q[I] = ld128<kNtLoad>(rq, hm.k_off[I] + sk);
      }
#pragma unroll
      for (int I = 0; I < 4; ++I) x.v[I] = ld128<kNtLoad>(rv, hm.v_off[I] + sv);
    }
    if constexpr (!FIXED) {
#pragma unroll
      for (int I = 0; I < 4; ++I) x.d[I] = ld128<kNtLoad>(rd, in4 ? tm.o4[I] : kOob, s4);
    }
#pragma unroll
    for (int I = 0; I < 8; ++I) x.gy[I] = ld128<kNtLoad>(rgy, in8 ? tm.o8[I] : kOob, s8);
    if constexpr (!FIXED) {
      const uint32_t s1 = static_cast<uint32_t>(t0) * 4u;
      x.p = ld128<false>(rp, in1 ? tm.o1 : kOob, s1);
      x.r = ld128<false>(rr, in1 ? tm.o1 : kOob, s1);
    }
  };
  auto put = [&](const Stage& x) __attribute__((always_inline)) {
    if constexpr (W) {
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        *reinterpret_cast<v4f*>(&tile[BwdTile::K + tm.s4[I]]) = x.k[I];
        *reinterpret_cast<v4f*>(&tile[BwdTile::Q + tm.s4[I]]) = x.q[I];
      }
#pragma unroll
      for (int I = 0; I < 8; ++I) *reinterpret_cast<v4f*>(&tile[BwdTile::V + tm.s8[I]]) = x.v[I];
    } else if constexpr (Q8) {
      const v4u wk = __builtin_bit_cast(v4u, x.k), wq = __builtin_bit_cast(v4u, x.q);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        *reinterpret_cast<v4f*>(&tile[BwdTile::K + qm.k_lds[u]]) = widen_f8<F>(wk[u]);
        *reinterpret_cast<v4f*>(&tile[BwdTile::Q + qm.k_lds[u]]) = widen_f8<F>(wq[u]);
      }
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        const v4u wv = __builtin_bit_cast(v4u, x.v[I]);
#pragma unroll
        for (int w = 0; w < 4; ++w) *reinterpret_cast<v4f*>(&tile[BwdTile::V + qm.v_lds[I][w]]) = widen_f8<F>(wv[w]);
      }
    } else {
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        *reinterpret_cast<v4f*>(&tile[BwdTile::K + hm.k_lds[I][0]]) = widen_lo(x.k[I]);
        *reinterpret_cast<v4f*>(&tile[BwdTile::K + hm.k_lds[I][1]]) = widen_hi(x.k[I]);
        *reinterpret_cast<v4f*>(&tile[BwdTile::Q + hm.k_lds[I][0]]) = widen_lo(x.q[I]);
        *reinterpret_cast<v4f*>(&tile[BwdTile::Q + hm.k_lds[I][1]]) = widen_hi(x.q[I]);
      }
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        *reinterpret_cast<v4f*>(&tile[BwdTile::V + hm.v_lds[I][0]]) = widen_lo(x.v[I]);
        *reinterpret_cast<v4f*>(&tile[BwdTile::V + hm.v_lds[I][1]]) = widen_hi(x.v[I]);
      }
    }
    if constexpr (!FIXED) {
#pragma unroll
      for (int I = 0; I < 4; ++I) *reinterpret_cast<v4f*>(&tile[BwdTile::D + tm.s4[I]]) = x.d[I];
    }
#pragma unroll
    for (int I = 0; I < 8; ++I) *reinterpret_cast<v4f*>(&tile[BwdTile::GY + tm.s8[I]]) = x.gy[I];
    if constexpr (!FIXED) {
      *reinterpret_cast<v4f*>(&tile[BwdTile::P + tm.s1]) = x.p;
      *reinterpret_cast<v4f*>(&tile[BwdTile::R + tm.s1]) = x.r;
    }
  };
  // Checkpoint record c into the CK region of slot tl, once the LDS reads of
  // the record that was there have completed.
  auto issue_ck = [&](float* tl, int64_t c) __attribute__((always_inline)) {
    lds_wait();
    const uint32_t cm = static_cast<uint32_t>(c) * 128u, cc = static_cast<uint32_t>(c) * 64u;
    dma16<kNtCkpt>(rbm, (tl + BwdTile::CK), ckoff.m0 + cm);
    dma16<kNtCkpt>(rbm, (tl + BwdTile::CK) + 256, ckoff.m1 + cm);
    dma16(rbc, (tl + BwdTile::CK) + 512, ckoff.c + cc);
  };
  auto take = [&](Out& o) __attribute__((always_inline)) {
    if constexpr (W) {
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        o.k[I] = *reinterpret_cast<const v4f*>(&tile[BwdTile::K + tm.s4[I]]);
        o.q[I] = *reinterpret_cast<const v4f*>(&tile[BwdTile::Q + tm.s4[I]]);
      }
#pragma unroll
      for (int I = 0; I < 8; ++I) o.v[I] = *reinterpret_cast<const v4f*>(&tile[BwdTile::V + tm.s8[I]]);
    } else if constexpr (Q8) {
      v4u wk, wq;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        wk[u] = narrow_f8<F>(*reinterpret_cast<const v4f*>(&tile[BwdTile::K + qm.k_lds[u]]));
        wq[u] = narrow_f8<F>(*reinterpret_cast<const v4f*>(&tile[BwdTile::Q + qm.k_lds[u]]));
      }
      o.k = __builtin_bit_cast(v4f, wk);
      o.q = __builtin_bit_cast(v4f, wq);
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        v4u wv;
#pragma unroll
        for (int w = 0; w < 4; ++w) wv[w] = narrow_f8<F>(*reinterpret_cast<const v4f*>(&tile[BwdTile::V + qm.v_lds[I][w]]));
        o.v[I] = __builtin_bit_cast(v4f, wv);
      }
    } else {
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        o.k[I] = narrow(*reinterpret_cast<const v4f*>(&tile[BwdTile::K + hm.k_lds[I][0]]),
                        *reinterpret_cast<const v4f*>(&tile[BwdTile::K + hm.k_lds[I][1]]));
        o.q[I] = narrow(*reinterpret_cast<const v4f*>(&tile[BwdTile::Q + hm.k_lds[I][0]]),
                        *reinterpret_cast<const v4f*>(&tile[BwdTile::Q + hm.k_lds[I][1]]));
      }
#pragma unroll
      for (int I = 0; I < 4; ++I)
        o.v[I] = narrow(*reinterpret_cast<const v4f*>(&tile[BwdTile::V + hm.v_lds[I][0]]),
                        *reinterpret_cast<const v4f*>(&tile[BwdTile::V + hm.v_lds[I][1]]));
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) o.d[I] = *reinterpret_cast<const v4f*>(&tile[BwdTile::D + tm.s4[I]]);
    o.p = *reinterpret_cast<const v4f*>(&tile[BwdTile::P + tm.s1]);
    o.r = *reinterpret_cast<const v4f*>(&tile[BwdTile::R + tm.s1]);
  };
  // Gradients of tile J; pieces of tokens at or past T are dropped.
  auto store_grads = [&](const Out& o, int64_t J) __attribute__((always_inline)) {
    const int64_t t0 = J * 2 * SUB;
    const uint32_t sk = static_cast<uint32_t>(t0 * e4), sv = static_cast<uint32_t>(t0 * e8);
    const uint32_t s4 = static_cast<uint32_t>(t0) * 16u, s8 = static_cast<uint32_t>(t0) * 32u;
    const bool in4 = t0 + tm.t4 < T, in8 = t0 + tm.t8 < T;
    if constexpr (W) {
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        st128<kNtStore>(rgk, o.k[I], in4 ? tm.o4[I] : kOob, s4);
        st128<kNtStore>(rgq, o.q[I], in4 ? tm.o4[I] : kOob, s4);
      }
#pragma unroll
      for (int I = 0; I < 8; ++I) st128<kNtStore>(rgv, o.v[I], in8 ? tm.o8[I] : kOob, s8);
    } else if constexpr (Q8) {
      const bool kin = t0 + qm.k_tok < T, vin = t0 + qm.v_tok < T;
      st128<kNtStore>(rgk, o.k, kin ? qm.k_off : kOob, sk);
      st128<kNtStore>(rgq, o.q, kin ? qm.k_off : kOob, sk);
#pragma unroll
      for (int I = 0; I < 2; ++I) st128<kNtStore>(rgv, o.v[I], vin ? qm.v_off[I] : kOob, sv);
    } else {
      const bool kin = t0 + hm.k_tok < T, vin = t0 + hm.v_tok < T;
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        st128<kNtStore>(rgk, o.k[I], kin ? hm.k_off[I] : kOob, sk);
        st128<kNtStore>(rgq, o.q[I], kin ? hm.k_off[I] : kOob, sk);
      }
#pragma unroll
      for (int I = 0; I < 4; ++I) st128<kNtStore>(rgv, o.v[I], vin ? hm.v_off[I] : kOob, sv);
    }
    if (a.gd) {
#pragma unroll
      for (int I = 0; I < 4; ++I) st128<kNtStore>(rgd, o.d[I], in4 ? tm.o4[I] : kOob, s4);
    }
    const uint32_t offp = t0 + tm.t1 < T ? tm.o1 : kOob, s1 = static_cast<uint32_t>(t0) * 4u;
    if (a.gp) st128(rgp, o.p, offp, s1);
    if (a.gr) st128(rgr, o.r, offp, s1);
  };
  auto chunk_len = [&](int64_t c) __attribute__((always_inline)) {
    return static_cast<int>((T - c * SUB) < SUB ? (T - c * SUB) : SUB);
  };
  // Chunk c from slot tl; the slot's checkpoint region then receives the
  // record of chunk c - 2 (the same slot's chunk in the next tile).
  auto run_chunk = [&](float* tl, int64_t c) __attribute__((always_inline)) {
    Bel b;
    bel_from_lds(b, tl + BwdTile::CK, s, g);
    if (c >= 2) issue_ck(tl, c - 2);
    core.run(tl, b, chunk_len(c));
  };
  // Tile J with one record (interval 16, in slot 0's checkpoint region): the
  // second chunk starts from the record advanced over the first chunk's 8
  // tokens, the first from the record itself; the region then receives the
  // record of tile J - 1.
  auto run_tile16 = [&](int64_t J) __attribute__((always_inline)) {
    if (2 * J + 1 < nsub) {
      Bel b;
      bel_from_lds(b, tile + BwdTile::CK, s, g);
      core.advance(tile, b);
      core.run(tile + BwdTile::SIZE, b, chunk_len(2 * J + 1));
    }
    Bel b0;
    bel_from_lds(b0, tile + BwdTile::CK, s, g);
    if (J > 0) issue_ck(tile, J - 1);
    core.run(tile, b0, chunk_len(2 * J));
  };

  // Tiles run from the last to the first.  At the start of tile J every
  // outstanding load was issued during tile J + 1 and is awaited; the
  // gradients of tile J + 1 are read out of LDS, the tile's staged inputs
  // written there, those gradients stored, the loads of tile J - 1 issued,
  // and chunks 2J + 1 and 2J replayed and reversed.
  Stage st;
  load(st, ntiles - 1);
  if constexpr (IV == SUB) {
    issue_ck(tile, 2 * (ntiles - 1));
    if (2 * ntiles - 1 < nb) issue_ck(tile + BwdTile::SIZE, 2 * ntiles - 1);
    else if (ntiles > 1) issue_ck(tile + BwdTile::SIZE, 2 * ntiles - 3);
  } else {
    issue_ck(tile, ntiles - 1);
  }
  for (int64_t J = ntiles - 1; J >= 0; --J) {
    Out go;
    vm_wait<0>();
    if (J + 1 < ntiles) take(go);
    __builtin_amdgcn_sched_barrier(0);
    put(st);
    __builtin_amdgcn_sched_barrier(0);
    if (J + 1 < ntiles) store_grads(go, J + 1);
    if (J > 0) load(st, J - 1);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (IV == SUB) {
      if (2 * J + 1 < nb) run_chunk(tile + BwdTile::SIZE, 2 * J + 1);
      run_chunk(tile, 2 * J);
    } else {
      run_tile16(J);
    }
  }
  {
    Out go;
    take(go);
    store_grads(go, 0);
  }
  core.store_initial(a.gm0, a.gc0, n0, valid, unit);
}

}  // namespace r4

// Launch helpers used by the dispatch in bssm_recurrence.hip.
hipError_t launch_forward_r4(bool fixed, const FwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + r4::SPW - 1) / r4::SPW;
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  switch (a.in_fmt) {
    case kInBf16:
      if (fixed) hipLaunchKernelGGL((r4::forward_kernel<true, kInBf16>), grid, block, 0, stream, a);
      else hipLaunchKernelGGL((r4::forward_kernel<false, kInBf16>), grid, block, 0, stream, a);
      break;
    case kInE4M3:
      if (fixed) hipLaunchKernelGGL((r4::forward_kernel<true, kInE4M3>), grid, block, 0, stream, a);
      else hipLaunchKernelGGL((r4::forward_kernel<false, kInE4M3>), grid, block, 0, stream, a);
      break;
    case kInE5M2:
      if (fixed) hipLaunchKernelGGL((r4::forward_kernel<true, kInE5M2>), grid, block, 0, stream, a);
      else hipLaunchKernelGGL((r4::forward_kernel<false, kInE5M2>), grid, block, 0, stream, a);
      break;
    default:
      if (fixed) hipLaunchKernelGGL((r4::forward_kernel<true, kInF32>), grid, block, 0, stream, a);
      else hipLaunchKernelGGL((r4::forward_kernel<false, kInF32>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

template <int IV>
hipError_t launch_backward_r4_iv(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + r4::SPW - 1) / r4::SPW;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWave);
  switch (a.in_fmt) {
    case kInBf16:
      if (fixed) hipLaunchKernelGGL((r4::backward_tile_kernel<true, false, kInBf16, IV>), grid, block, 0, stream, a);
      else if (dyn) hipLaunchKernelGGL((r4::backward_tile_kernel<false, true, kInBf16, IV>), grid, block, 0, stream, a);
      else hipLaunchKernelGGL((r4::backward_tile_kernel<false, false, kInBf16, IV>), grid, block, 0, stream, a);
      break;
    case kInE4M3:
      if (fixed) hipLaunchKernelGGL((r4::backward_tile_kernel<true, false, kInE4M3, IV>), grid, block, 0, stream, a);
      else if (dyn) hipLaunchKernelGGL((r4::backward_tile_kernel<false, true, kInE4M3, IV>), grid, block, 0, stream, a);
      else hipLaunchKernelGGL((r4::backward_tile_kernel<false, false, kInE4M3, IV>), grid, block, 0, stream, a);
      break;
    case kInE5M2:
      if (fixed) hipLaunchKernelGGL((r4::backward_tile_kernel<true, false, kInE5M2, IV>), grid, block, 0, stream, a);
      else if (dyn) hipLaunchKernelGGL((r4::backward_tile_kernel<false, true, kInE5M2, IV>), grid, block, 0, stream, a);
      else hipLaunchKernelGGL((r4::backward_tile_kernel<false, false, kInE5M2, IV>), grid, block, 0, stream, a);
      break;
    default:
      if (fixed) hipLaunchKernelGGL((r4::backward_tile_kernel<true, false, kInF32, IV>), grid, block, 0, stream, a);
      else if (dyn) hipLaunchKernelGGL((r4::backward_tile_kernel<false, true, kInF32, IV>), grid, block, 0, stream, a);
      else hipLaunchKernelGGL((r4::backward_tile_kernel<false, false, kInF32, IV>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

// Checkpoint chunk kRot4Chunk or twice that (checked by the C ABI).
hipError_t launch_backward_r4(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.n + r4::SPW - 1) / r4::SPW;
  if (blocks == 0) return hipSuccess;
  if (a.chunk == 2 * kRot4Chunk) return launch_backward_r4_iv<2 * kRot4Chunk>(fixed, dyn, a, stream);
  if (a.chunk != kRot4Chunk) return hipErrorInvalidValue;
  return launch_backward_r4_iv<kRot4Chunk>(fixed, dyn, a, stream);
}

}  // namespace bssm
