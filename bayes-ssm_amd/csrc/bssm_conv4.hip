// Length-four causal depthwise filter (CausalDepthwise4,
// example/train_6layer.py:160-191) on channels-last rows, gfx950.
//
// The mixer applies the filter to each projected stream [B, T, C] through a
// transposed view (train_6layer.py:474-480), so in memory every token is a
// row of C channels.  For channel c and token t,
//   y[t] = w[c,0] x[t-3] + w[c,1] x[t-2] + w[c,2] x[t-1] + w[c,3] x[t]
// with x = 0 before the sequence start.  A thread owns one 16-byte channel
// group (8 bf16 or 4 float32 channels) and streams it along a segment of
// tokens with the last three rows in registers, so each element is read and
// written once (plus a three-row halo per segment); consecutive lanes take
// consecutive groups of the same row.  The rows of one batch entry are
// addressed through a buffer descriptor whose range ends at token T, so the
// causal zero padding (tokens below 0, whose offsets wrap past the range) and
// the tail come from the hardware's range check.
//
// Block: 4 waves, one batch entry b, 64 channel groups; wave w takes the
// segments w, w + 4, ... of kSeg tokens.  The backward (gx[s] = sum_j
// w[c,j] gy[s+3-j], gw[c,j] = sum_t gy[t] x[t-3+j]) sums the weight gradient
// of its segments in registers, reduces the block's 4 waves in LDS and
// writes one partial row per (b, channel): grad_weight_partials [B, C, 4].

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "bssm_recurrence.h"

// Device scratch of the allocation-free backward (launch_conv4_backward_noalloc):
// the per-batch-entry weight-gradient partials [B, C, 4] of one call, reduced
// over B by a second kernel on the same stream.  Every GPU holds its own copy
// until the process ends; host code reaches it only through the address that
// hipGetSymbolAddress returns for the current device (conv4_scratch below),
// never through the name itself.  Calls that overlap on one GPU share it and
// race; each call rewrites every slot it reads, so nothing needs clearing.
static __device__ __align__(256) float scratch[bssm::kConv4ScratchFloats];

namespace bssm {
namespace conv4 {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t Rsrc;

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kSeg = 64;   // tokens per segment
constexpr int kStep = 8;   // rows loaded ahead within a segment
constexpr uint32_t kDword3 = 0x00020000;

__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kDword3);
}
__device__ __forceinline__ v4u ld16(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0));
}
__device__ __forceinline__ void st16(Rsrc r, v4u x, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(x, r, static_cast<int>(off), 0, 0);
}

// A 16-byte group as float32 values, and back.
template <typename T>
struct Group;
template <>
struct Group<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void widen(v4u p, float (&x)[4]) {
    const v4f f = __builtin_bit_cast(v4f, p);
    x[0] = f.x;
    x[1] = f.y;
    x[2] = f.z;
    x[3] = f.w;
  }
  __device__ __forceinline__ static v4u narrow(const float (&x)[4]) {
    const v4f f = {x[0], x[1], x[2], x[3]};
    return __builtin_bit_cast(v4u, f);
  }
};
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
template <>
struct Group<__bf16> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void widen(v4u p, float (&x)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __builtin_bit_cast(float, p[i] << 16);
      x[2 * i + 1] = __builtin_bit_cast(float, p[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static v4u narrow(const float (&x)[8]) {
    v4u p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf2 v;
      v[0] = static_cast<__bf16>(x[2 * i]);
      v[1] = static_cast<__bf16>(x[2 * i + 1]);
      p[i] = __builtin_bit_cast(uint32_t, v);
    }
    return p;
  }
};

template <typename T>
struct Lane {
  static constexpr int N = Group<T>::N;
  int64_t b, g;     // batch entry, channel group
  bool active;      // the group exists (C / N groups)
  uint32_t col;     // byte offset of the group within a row
  float w[N][4];
  __device__ __forceinline__ Lane(const ConvArgs& a) {
    const int64_t groups = a.c / N;
    const int64_t cblocks = (groups + kWave - 1) / kWave;
    b = blockIdx.x / cblocks;
    g = (blockIdx.x % cblocks) * kWave + (threadIdx.x & (kWave - 1));
    active = g < groups;
    const int64_t gc = active ? g : 0;
    col = static_cast<uint32_t>(gc * 16);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const v4f wi = *reinterpret_cast<const v4f*>(a.w + (gc * N + i) * 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) w[i][j] = wi[j];
    }
  }
};

template <typename T>
__global__ __launch_bounds__(kWave * kWaves) void forward_kernel(ConvArgs a) {
  constexpr int N = Group<T>::N;
  const Lane<T> L(a);
  if (!L.active) return;
  const int64_t T_ = a.t;
  const uint32_t rx = static_cast<uint32_t>(a.ldx * sizeof(T)), ry = static_cast<uint32_t>(a.c * sizeof(T));
  const Rsrc X = make_rsrc(reinterpret_cast<const char*>(a.x) + L.b * T_ * rx, static_cast<uint32_t>(T_) * rx);
  const Rsrc Y = make_rsrc(reinterpret_cast<const char*>(a.y) + L.b * T_ * ry, static_cast<uint32_t>(T_) * ry);
  const int64_t segs = (T_ + kSeg - 1) / kSeg;
  for (int64_t seg = threadIdx.x / kWave; seg < segs; seg += kWaves) {
    const int64_t t0 = seg * kSeg;
    // The three rows before the segment (zeros before token 0: the offsets
    // wrap past the range).
    float h[3][N];
#pragma unroll
    for (int k = 0; k < 3; ++k)
      Group<T>::widen(ld16(X, static_cast<uint32_t>(t0 - 3 + k) * rx + L.col), h[k]);
    for (int s = 0; s < kSeg; s += kStep) {
      if (t0 + s >= T_) break;
      v4u raw[kStep];
#pragma unroll
      for (int k = 0; k < kStep; ++k) raw[k] = ld16(X, static_cast<uint32_t>(t0 + s + k) * rx + L.col);
#pragma unroll
      for (int k = 0; k < kStep; ++k) {
        float x[N], y[N];
        Group<T>::widen(raw[k], x);
#pragma unroll
        for (int i = 0; i < N; ++i) {
          y[i] = fmaf(L.w[i][3], x[i], fmaf(L.w[i][2], h[2][i], fmaf(L.w[i][1], h[1][i], L.w[i][0] * h[0][i])));
          h[0][i] = h[1][i];
          h[1][i] = h[2][i];
          h[2][i] = x[i];
        }
        st16(Y, Group<T>::narrow(y), static_cast<uint32_t>(t0 + s + k) * ry + L.col);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kWave * kWaves) void backward_kernel(ConvArgs a) {
  constexpr int N = Group<T>::N;
  __shared__ float red[kWaves - 1][kWave][N * 4];
  const Lane<T> L(a);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int64_t T_ = a.t;
  const uint32_t rx = static_cast<uint32_t>(a.ldx * sizeof(T)), rc = static_cast<uint32_t>(a.c * sizeof(T));
  const Rsrc X = make_rsrc(reinterpret_cast<const char*>(a.x) + L.b * T_ * rx, static_cast<uint32_t>(T_) * rx);
  const Rsrc GY = make_rsrc(reinterpret_cast<const char*>(a.gy) + L.b * T_ * rc, static_cast<uint32_t>(T_) * rc);
  const uint32_t rgx = static_cast<uint32_t>((a.ldgx ? a.ldgx : a.c) * sizeof(T));
  const Rsrc GX = make_rsrc(reinterpret_cast<char*>(a.gx) + L.b * T_ * rgx, static_cast<uint32_t>(T_) * rgx);
  float gw[N][4];
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) gw[i][j] = 0.f;
  const int64_t segs = (T_ + kSeg - 1) / kSeg;
  if (L.active) {
    for (int64_t seg = wave; seg < segs; seg += kWaves) {
      const int64_t t0 = seg * kSeg;
      // Window: x[t-3..t-1] behind the token, gy[t+1..t+3] ahead of it.
      float hx[3][N], gq[3][N];
#pragma unroll
      for (int k = 0; k < 3; ++k) Group<T>::widen(ld16(X, static_cast<uint32_t>(t0 - 3 + k) * rx + L.col), hx[k]);
      float g0[N];
      Group<T>::widen(ld16(GY, static_cast<uint32_t>(t0) * rc + L.col), g0);
#pragma unroll
      for (int k = 0; k < 3; ++k)
        Group<T>::widen(ld16(GY, static_cast<uint32_t>(t0 + 1 + k) * rc + L.col), gq[k]);
      for (int s = 0; s < kSeg; s += kStep) {
        if (t0 + s >= T_) break;
        v4u rawx[kStep], rawg[kStep];
#pragma unroll
        for (int k = 0; k < kStep; ++k) {
          rawx[k] = ld16(X, static_cast<uint32_t>(t0 + s + k) * rx + L.col);
          rawg[k] = ld16(GY, static_cast<uint32_t>(t0 + s + k + 4) * rc + L.col);
        }
#pragma unroll
        for (int k = 0; k < kStep; ++k) {
          float x[N], g4[N], gx[N];
          Group<T>::widen(rawx[k], x);
          Group<T>::widen(rawg[k], g4);
#pragma unroll
          for (int i = 0; i < N; ++i) {
            // Token s' = t0 + s + k: gy[s'] = g0, gy[s'+1..s'+3] = gq, x[s'-3..s'-1] = hx.
            gx[i] = fmaf(L.w[i][0], gq[2][i], fmaf(L.w[i][1], gq[1][i], fmaf(L.w[i][2], gq[0][i], L.w[i][3] * g0[i])));
            gw[i][0] = fmaf(g0[i], hx[0][i], gw[i][0]);
            gw[i][1] = fmaf(g0[i], hx[1][i], gw[i][1]);
            gw[i][2] = fmaf(g0[i], hx[2][i], gw[i][2]);
            gw[i][3] = fmaf(g0[i], x[i], gw[i][3]);
            hx[0][i] = hx[1][i];
            hx[1][i] = hx[2][i];
            hx[2][i] = x[i];
            g0[i] = gq[0][i];
            gq[0][i] = gq[1][i];
            gq[1][i] = gq[2][i];
            gq[2][i] = g4[i];
          }
          st16(GX, Group<T>::narrow(gx), static_cast<uint32_t>(t0 + s + k) * rgx + L.col);
        }
      }
    }
  }
  // Weight gradient: waves 1..3 hand their sums to wave 0 through LDS.
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave - 1][lane][i * 4 + j] = gw[i][j];
  }
  __syncthreads();
  if (wave == 0 && L.active) {
#pragma unroll
    for (int w = 0; w < kWaves - 1; ++w)
#pragma unroll
      for (int i = 0; i < N; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) gw[i][j] += red[w][lane][i * 4 + j];
    float* out = a.gw_part + (L.b * a.c + L.g * N) * 4;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      v4f v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = gw[i][j];
      *reinterpret_cast<v4f*>(out + i * 4) = v;
    }
  }
}

// Sum over the batch of the partials [B, C * 4]: one thread per (channel,
// tap), four interleaved accumulators, a fixed order (deterministic).
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ part,
                                                              float* __restrict__ gw, int64_t b, int64_t cw) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= cw) return;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int64_t k = 0;
  for (; k + 4 <= b; k += 4) {
    s0 += part[(k + 0) * cw + i];
    s1 += part[(k + 1) * cw + i];
    s2 += part[(k + 2) * cw + i];
    s3 += part[(k + 3) * cw + i];
  }
  for (; k < b; ++k) s0 += part[k * cw + i];
  gw[i] = (s0 + s1) + (s2 + s3);
}

// Column sums over the T rows of each batch entry of a bf16 [B, T, cols]
// view with row stride ld: out [B, cols] (float32).  A lane owns a column
// pair (one 4-byte load per row, a wave reading 256 contiguous bytes of a
// row); the block's 4 waves take every 4th row and meet in LDS.
__global__ __launch_bounds__(256) void column_sums_kernel(const uint32_t* __restrict__ x, int64_t ld2, int64_t t,
                                                          int64_t pairs, float* __restrict__ out) {
  __shared__ float red[kWaves - 1][kWave][2];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int64_t b = blockIdx.y;
  const int64_t cp = static_cast<int64_t>(blockIdx.x) * kWave + lane;
  const bool active = cp < pairs;
  const uint32_t* row = x + b * t * ld2 + (active ? cp : 0);
  float s0 = 0.f, s1 = 0.f;
  if (active) {
    // Eight rows' loads in flight before their sums.
    constexpr int kAhead = 8;
    int64_t r = wave;
    for (; r + (kAhead - 1) * kWaves < t; r += kAhead * kWaves) {
      uint32_t w[kAhead];
#pragma unroll
      for (int i = 0; i < kAhead; ++i) w[i] = row[(r + i * kWaves) * ld2];
#pragma unroll
      for (int i = 0; i < kAhead; ++i) {
        s0 += __builtin_bit_cast(float, w[i] << 16);
        s1 += __builtin_bit_cast(float, w[i] & 0xffff0000u);
      }
    }
    for (; r < t; r += kWaves) {
      const uint32_t w = row[r * ld2];
      s0 += __builtin_bit_cast(float, w << 16);
      s1 += __builtin_bit_cast(float, w & 0xffff0000u);
    }
  }
  if (wave > 0) {
    red[wave - 1][lane][0] = s0;
    red[wave - 1][lane][1] = s1;
  }
  __syncthreads();
  if (wave == 0 && active) {
#pragma unroll
    for (int k = 0; k < kWaves - 1; ++k) {
      s0 += red[k][lane][0];
      s1 += red[k][lane][1];
    }
    out[b * 2 * pairs + 2 * cp] = s0;
    out[b * 2 * pairs + 2 * cp + 1] = s1;
  }
}

// Column sums of up to three row-major float32 matrices in one launch (the
// block's weight-gradient partials), written float32 or bf16 (round to
// nearest even).  A block takes w = 32 columns (8 for narrower matrices) of
// one matrix; its 256 / w row groups sum every (256 / w)-th row, four loads in
// flight, and meet in LDS in a fixed order.
__global__ __launch_bounds__(256) void fold_kernel(FoldArgs a) {
  __shared__ float red[256];
  int m = 0;
  while (m + 1 < a.count && static_cast<int64_t>(blockIdx.x) >= a.first[m + 1]) ++m;
  const int64_t cols = a.cols[m], rows = a.rows[m];
  const int w = cols >= 32 ? 32 : 8, groups = 256 / w;
  const int cl = threadIdx.x % w, g = threadIdx.x / w;
  const int64_t c = (static_cast<int64_t>(blockIdx.x) - a.first[m]) * w + cl;
  const float* p = a.part[m];
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (c < cols) {
    int64_t r = g;
    for (; r + 3 * groups < rows; r += 4 * groups) {
      s0 += p[r * cols + c];
      s1 += p[(r + groups) * cols + c];
      s2 += p[(r + 2 * groups) * cols + c];
      s3 += p[(r + 3 * groups) * cols + c];
    }
    for (; r < rows; r += groups) s0 += p[r * cols + c];
  }
  red[threadIdx.x] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (g == 0 && c < cols) {
    float s = red[cl];
    for (int k = 1; k < groups; ++k) s += red[k * w + cl];
    if (a.bf16) static_cast<__bf16*>(a.out[m])[c] = static_cast<__bf16>(s);
    else static_cast<float*>(a.out[m])[c] = s;
  }
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
hipError_t conv4_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch[dev] = static_cast<float*>(p);
  }
  *out = g_scratch[dev];
  return hipSuccess;
}

}  // namespace
}  // namespace conv4

hipError_t launch_conv4_backward_noalloc(const ConvArgs& args, float* grad_weight, hipStream_t stream) {
  float* part = nullptr;
  hipError_t e = conv4::conv4_scratch(&part);
  if (e != hipSuccess) return e;
  ConvArgs a = args;
  a.gw_part = part;
  // Writes every [b, c, 4] slot the reduction reads (zeros when T = 0).
  e = launch_conv4_backward(a, stream);
  if (e != hipSuccess) return e;
  const int64_t cw = a.c * 4;
  if (cw == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((cw + 255) / 256)), block(256);
  hipLaunchKernelGGL(conv4::reduce_partials_kernel, grid, block, 0, stream, part, grad_weight, a.b, cw);
  return hipGetLastError();
}

hipError_t launch_column_sums_bf16(const void* x, int64_t ld, int64_t b, int64_t t, int64_t cols, float* out,
                                  hipStream_t stream) {
  const int64_t pairs = cols / 2;
  if (b == 0 || pairs == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((pairs + conv4::kWave - 1) / conv4::kWave), static_cast<unsigned>(b));
  hipLaunchKernelGGL(conv4::column_sums_kernel, grid, dim3(conv4::kWave * conv4::kWaves), 0, stream,
                     static_cast<const uint32_t*>(x), ld / 2, t, pairs, out);
  return hipGetLastError();
}

hipError_t launch_fold(FoldArgs a, hipStream_t stream) {
  int64_t blocks = 0;
  for (int i = 0; i < a.count; ++i) {
    a.first[i] = blocks;
    const int64_t w = a.cols[i] >= 32 ? 32 : 8;
    blocks += (a.cols[i] + w - 1) / w;
  }
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(conv4::fold_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_conv4_forward(const ConvArgs& a, hipStream_t stream) {
  const int64_t n = a.bf16 ? 8 : 4;
  const int64_t blocks = a.b * ((a.c / n + conv4::kWave - 1) / conv4::kWave);
  if (blocks == 0 || a.t == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(conv4::kWave * conv4::kWaves);
  if (a.bf16) hipLaunchKernelGGL(conv4::forward_kernel<__bf16>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(conv4::forward_kernel<float>, grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_conv4_backward(const ConvArgs& a, hipStream_t stream) {
  const int64_t n = a.bf16 ? 8 : 4;
  const int64_t blocks = a.b * ((a.c / n + conv4::kWave - 1) / conv4::kWave);
  if (blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(blocks)), block(conv4::kWave * conv4::kWaves);
  if (a.bf16) hipLaunchKernelGGL(conv4::backward_kernel<__bf16>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(conv4::backward_kernel<float>, grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace bssm
