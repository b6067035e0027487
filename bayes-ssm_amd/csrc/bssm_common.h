// Device primitives shared by the gfx950 Bayesian-recurrence kernels.
//
// Work decomposition used by every recurrence kernel: one wave64 per
// workgroup; a *group* of G adjacent lanes owns one sequence.  Inside a group
// the value columns of the mean are split into contiguous blocks of M/G
// columns per lane, and the covariance rows are split round-robin
// (row r lives in lane r % G when D >= G; with D < G the rows are replicated
// and lane g owns row g % D).  All cross-lane traffic inside a group uses DPP
// (quad permutes / half-row mirror) so it stays on the VALU and never touches
// LDS or memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bssm {

constexpr int kWave = 64;

// Native 4-float vector (the builtins below need a plain vector type).
typedef float v4f __attribute__((ext_vector_type(4)));

// Streamed data is touched once per pass.  Tile rows that cover whole
// 128-byte lines use nontemporal accesses (no L2 retention); shorter row
// segments (e.g. 8 tokens of a per-token scalar = 32 bytes) use ordinary
// accesses so the rest of the line stays in L2 for the neighbouring tiles.
// The byte thresholds are measured tuning choices.
#ifndef BSSM_NT_LOAD_MIN
#define BSSM_NT_LOAD_MIN 128
#endif
#ifndef BSSM_NT_STORE_MIN
#define BSSM_NT_STORE_MIN 128
#endif
template <bool NT>
__device__ __forceinline__ v4f load_stream(const float* p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p));
  else return *reinterpret_cast<const v4f*>(p);
}
template <bool NT>
__device__ __forceinline__ void store_stream(float* p, v4f v) {
  if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(p));
  else *reinterpret_cast<v4f*>(p) = v;
}

// ---------------------------------------------------------------- DPP moves
// dpp_ctrl encodings (gfx9 family): quad_perm = 8-bit lane selector,
// row_shl/shr/ror = 0x100 + n, row_mirror = 0x140, row_half_mirror = 0x141.
// Every pattern used here (quad permutes, half-row mirror) reads a valid
// lane for every lane, so bound_ctrl never takes effect; setting it (with a
// zero `old`) lets the compiler fold the move into the consuming VALU op
// (v_add_f32_dpp and the like).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

constexpr int quad_perm(int a, int b, int c, int d) { return a | (b << 2) | (c << 4) | (d << 6); }
constexpr int kXor1 = quad_perm(1, 0, 3, 2);
constexpr int kXor2 = quad_perm(2, 3, 0, 1);
constexpr int kHalfMirror = 0x141;  // lane l <- lane 7-l inside each 8-lane half-row

// Value of lane (l ^ (1 << B)).  B = 0, 1 are single DPP quad permutes; B = 2
// (8-lane groups) goes through the cross-lane permute unit.
template <int B>
__device__ __forceinline__ float xor_lane(float x) {
  if constexpr (B == 0) return dpp<kXor1>(x);
  else if constexpr (B == 1) return dpp<kXor2>(x);
  else return __shfl_xor(x, 1 << B, kWave);
}

// Sum over the G lanes of the caller's group; every lane of the group gets
// the bitwise-identical result (each step adds two commuted operands).
template <int G>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8, "group size");
  if constexpr (G >= 2) x += dpp<kXor1>(x);
  if constexpr (G >= 4) x += dpp<kXor2>(x);
  if constexpr (G >= 8) x += dpp<kHalfMirror>(x);
  return x;
}

// Value held by lane SRC of the caller's group.
template <int G, int SRC>
__device__ __forceinline__ float group_bcast(float x, int lane) {
  static_assert(SRC >= 0 && SRC < G, "source lane");
  if constexpr (G == 1) {
    return x;
  } else if constexpr (G == 2) {
    return dpp<quad_perm(SRC, SRC, 2 + SRC, 2 + SRC)>(x);
  } else if constexpr (G == 4) {
    return dpp<quad_perm(SRC, SRC, SRC, SRC)>(x);
  } else {
    // Broadcast inside each quad, then take the mirrored half for the quad
    // that does not contain SRC.
    constexpr int q = SRC & 3;
    const float y = dpp<quad_perm(q, q, q, q)>(x);
    const float z = dpp<kHalfMirror>(y);
    return (((lane >> 2) & 1) == (SRC >> 2)) ? y : z;
  }
}

// ------------------------------------------------------ row/column ownership
template <int D, int M, int G>
struct Layout {
  static_assert(M % G == 0, "value columns must split evenly over the group");
  static constexpr int SPW = kWave / G;             // sequences per wave
  static constexpr int CPL = M / G;                 // value columns per lane
  static constexpr int RPL = (D >= G) ? D / G : 1;  // covariance rows per lane
  static constexpr int OWNERS = (D >= G) ? G : D;   // lanes that own distinct rows
  // Row of slot jj for lane g.
  static __device__ __forceinline__ int row(int g, int jj) { return (D >= G) ? g + G * jj : g % D; }
  // Lane (within the group) and slot holding row r.
  static constexpr int owner(int r) { return (D >= G) ? r % G : r; }
  static constexpr int slot(int r) { return (D >= G) ? r / G : 0; }
  // Lanes that write per-row outputs (one writer per row).
  static __device__ __forceinline__ bool row_writer(int g) { return (D >= G) || g < D; }
};

// Per-lane register arrays: own covariance rows, and all rows x own columns.
template <int D, int M, int G>
using RowsArr = float[Layout<D, M, G>::RPL][D];
template <int D, int M, int G>
using ColsArr = float[D][Layout<D, M, G>::CPL];
template <int D, int M, int G>
using OwnRowVec = float[Layout<D, M, G>::RPL];

// Every lane contributes a partial x[r] for each row r; returns the group
// total of the lane's own rows (own[jj] = sum over lanes of x[row(g, jj)]).
// Recursive halving: log2(min(G, D)) exchange stages, then plain all-reduce
// stages when rows are replicated (G > D).
template <int D, int G>
__device__ __forceinline__ void group_reduce_rows(const float (&x)[D], float (&own)[(D >= G) ? D / G : 1],
                                                  int g) {
  if constexpr (D == 8 && G == 8) {
    // Eight lanes, one row each (row g): halve on the top lane bit first, so
    // that its partner can be the half-row mirror (lane 7 - g, which also
    // differs in bit 2) and every exchange stays a DPP move.  Stage k splits
    // the rows still held on bit (2 - k) of the row index; the partner holds
    // the same rows and keeps the other half.
    float cur[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) cur[r] = x[r];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int half = 4 >> k;
      const bool hi = (g >> (2 - k)) & 1;
#pragma unroll
      for (int m = 0; m < half; ++m) {
        // Both halves summed with the partner's copy (two DPP adds), one select.
        float lo, up;
        if (k == 0) {
          lo = cur[m] + dpp<kHalfMirror>(cur[m]);
          up = cur[half + m] + dpp<kHalfMirror>(cur[half + m]);
        } else if (k == 1) {
          lo = cur[m] + xor_lane<1>(cur[m]);
          up = cur[half + m] + xor_lane<1>(cur[half + m]);
        } else {
          lo = cur[m] + xor_lane<0>(cur[m]);
          up = cur[half + m] + xor_lane<0>(cur[half + m]);
        }
        cur[m] = hi ? up : lo;
      }
    }
    own[0] = cur[0];
    return;
  }
  constexpr int RS = (D >= G) ? G : D;  // lanes taking part in the scatter
  float cur[D];
#pragma unroll
  for (int r = 0; r < D; ++r) cur[r] = x[r];
  int width = D;
#pragma unroll
  for (int b = 0; (1 << b) < RS; ++b) {
    const bool hi = (g >> b) & 1;
#pragma unroll
    for (int m = 0; m < D / 2; ++m) {
      if (2 * m + 1 < width) {
        const float lo_v = cur[2 * m], hi_v = cur[2 * m + 1];
        const float send = hi ? lo_v : hi_v;
        const float keep = hi ? hi_v : lo_v;
        float recv;
        if (b == 0) recv = xor_lane<0>(send);
        else if (b == 1) recv = xor_lane<1>(send);
        else recv = xor_lane<2>(send);
        cur[m] = keep + recv;
      }
    }
    width >>= 1;
  }
  if constexpr (G > D) {
    // Replicated rows: finish with an all-reduce over the copies.
#pragma unroll
    for (int b = 0; (1 << b) < G; ++b) {
      if ((1 << b) >= D) {
        if (b == 0) cur[0] += xor_lane<0>(cur[0]);
        else if (b == 1) cur[0] += xor_lane<1>(cur[0]);
        else cur[0] += xor_lane<2>(cur[0]);
      }
    }
  }
#pragma unroll
  for (int jj = 0; jj < ((D >= G) ? D / G : 1); ++jj) own[jj] = cur[jj];
}

__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// ---------------------------------------------------------- tile staging
// A tile holds TT tokens of SPW sequences for one stream of W floats per
// token.  In LDS, sequence s occupies [s * stride, s * stride + TT * W) with
// stride = TT * W + 4, so per-token reads of 16 different sequences do not
// land in the same LDS banks.
template <int W, int TT>
struct Tile {
  static constexpr int PER = TT * W;
  static constexpr int STRIDE = PER + 4;
};

// This lane's share of one tile of one stream, held in registers between
// the global loads and the LDS commit.  Every load of a tile is issued before
// any of them is consumed, so a tile costs one memory latency, and a tile can
// be loaded while the previous one is being computed.  Element e (a multiple
// of 4) of the tile belongs to lane (e / 4) % 64; rows past N and tokens past
// len read as zero so idle lanes compute on finite data.  Requires every
// 4-float group to be 16-byte aligned (checked by the caller).
template <int W, int TT, int SPW>
struct TileRegs {
  using T_ = Tile<W, TT>;
  static constexpr int TOTAL = SPW * T_::PER;
  static constexpr int NV = (TOTAL + 4 * kWave - 1) / (4 * kWave);
  // One wave instruction covers 4 * 64 floats = SEQ_STEP whole sequence rows,
  // so lane l always holds column o0 of rows s0 + it * SEQ_STEP: one lane
  // offset, and a wave-uniform base that advances per instruction.
  static constexpr int SEQ_STEP = 4 * kWave / T_::PER;
  static_assert(T_::PER % 4 == 0 && (4 * kWave) % T_::PER == 0, "tile rows must divide a wave instruction");
  v4f r[NV];

  // Rows of one tile are `row` floats apart in global memory (row = T * W).
  __device__ __forceinline__ void load(const float* __restrict__ g, int64_t n0, int64_t n, int64_t t, int64_t t0,
                                       int len, int lane) {
    const int s0 = (lane * 4) / T_::PER, o0 = (lane * 4) % T_::PER;
    const int64_t row = t * W;
    const float* base = g + n0 * row + t0 * W;
    const uint32_t off = static_cast<uint32_t>(s0) * static_cast<uint32_t>(row) + static_cast<uint32_t>(o0);
    const bool col_ok = o0 < len * W;
#pragma unroll
    for (int it = 0; it < NV; ++it) {
      const int s = s0 + it * SEQ_STEP;
      v4f val = {0.f, 0.f, 0.f, 0.f};
      if (s < SPW && col_ok && n0 + s < n)
        val = load_stream<(T_::PER * 4 >= BSSM_NT_LOAD_MIN)>(base + static_cast<int64_t>(it * SEQ_STEP) * row + off);
      r[it] = val;
    }
  }

  __device__ __forceinline__ void commit(float* __restrict__ lds, int lane) const {
    const int s0 = (lane * 4) / T_::PER, o0 = (lane * 4) % T_::PER;
    float* dst = lds + s0 * T_::STRIDE + o0;
#pragma unroll
    for (int it = 0; it < NV; ++it) {
      if (s0 + it * SEQ_STEP < SPW)
        *reinterpret_cast<v4f*>(dst + it * SEQ_STEP * T_::STRIDE) = r[it];
    }
  }
};

// Scalar global -> LDS copy of one tile, for streams whose rows are not
// 16-byte aligned (T * W not a multiple of 4, or an unaligned base pointer).
// A compact rolled loop: this is the rarely used fallback, kept small so it
// does not inflate the register budget of the fast path.
template <int W, int TT, int SPW>
__device__ __forceinline__ void stage_in_scalar(float* __restrict__ lds, const float* __restrict__ g, int64_t n0,
                                                int64_t n, int64_t t, int64_t t0, int len, int lane) {
  using T_ = Tile<W, TT>;
  constexpr int TOTAL = SPW * T_::PER;
  const int valid = len * W;
#pragma unroll 1
  for (int e = lane; e < TOTAL; e += kWave) {
    const int s = e / T_::PER, o = e - s * T_::PER;
    lds[s * T_::STRIDE + o] = (n0 + s < n && o < valid) ? g[((n0 + s) * t + t0) * W + o] : 0.f;
  }
}

// Register-staged copy of one tile (loads, then LDS commit).
template <int W, int TT, int SPW>
__device__ __forceinline__ void stage_in(float* __restrict__ lds, const float* __restrict__ g, int64_t n0,
                                         int64_t n, int64_t t, int64_t t0, int len, bool vec, int lane) {
  if (vec) {
    TileRegs<W, TT, SPW> regs;
    regs.load(g, n0, n, t, t0, len, lane);
    regs.commit(lds, lane);
  } else {
    stage_in_scalar<W, TT, SPW>(lds, g, n0, n, t, t0, len, lane);
  }
}

// LDS -> global copy of the first len tokens of a tile.
template <int W, int TT, int SPW>
__device__ __forceinline__ void stage_out(const float* __restrict__ lds, float* __restrict__ g, int64_t n0,
                                          int64_t n, int64_t t, int64_t t0, int len, bool vec, int lane) {
  using T_ = Tile<W, TT>;
  constexpr int TOTAL = SPW * T_::PER;
  const int valid = len * W;
  if (vec) {
    using R = TileRegs<W, TT, SPW>;
    const int s0 = (lane * 4) / T_::PER, o0 = (lane * 4) % T_::PER;
    const int64_t row = t * W;
    float* base = g + n0 * row + t0 * W;
    const uint32_t off = static_cast<uint32_t>(s0) * static_cast<uint32_t>(row) + static_cast<uint32_t>(o0);
    const float* src = lds + s0 * T_::STRIDE + o0;
#pragma unroll
    for (int it = 0; it < R::NV; ++it) {
      const int s = s0 + it * R::SEQ_STEP;
      if (s < SPW && o0 < valid && n0 + s < n) {
        float* dst = base + static_cast<int64_t>(it * R::SEQ_STEP) * row + off;
        const float* lsrc = src + it * R::SEQ_STEP * T_::STRIDE;
        if (o0 + 4 <= valid) {
          store_stream<(T_::PER * 4 >= BSSM_NT_STORE_MIN)>(dst, *reinterpret_cast<const v4f*>(lsrc));
        } else {
          // The group straddles the end of the tile: the floats past `valid`
          // belong to the next tile's tokens and must not be overwritten.
          for (int e = 0; e < valid - o0; ++e) dst[e] = lsrc[e];
        }
      }
    }
  } else {
#pragma unroll 1
    for (int e = lane; e < TOTAL; e += kWave) {
      const int s = e / T_::PER, o = e - s * T_::PER;
      if (n0 + s < n && o < valid) g[((n0 + s) * t + t0) * W + o] = lds[s * T_::STRIDE + o];
    }
  }
}

}  // namespace bssm
