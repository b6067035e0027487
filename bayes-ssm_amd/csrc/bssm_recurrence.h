// Internal launch interface between the C ABI (bssm_capi.hip) and the
// recurrence kernels (bssm_recurrence.hip).
#pragma once

#include "bssm_fp8.h"

#include "bssm_common.h"

namespace bssm {

struct FwdArgs {
  const float* k;
  const float* v;
  const float* q;
  const float* d;
  const float* p;
  const float* r;
  const float* m0;
  const float* c0;
  float* y;
  float* mT;
  float* cT;
  float* bm;
  float* bc;
  int64_t n;
  int64_t t;
  int64_t chunk;
  int64_t nb;
  float floor;
  int vec_kqd, vec_v, vec_pr;  // 16-byte staging allowed per stream class
  int rot4;                    // D = 4 rotated-layout kernels allowed (see bssm_rot4.hip)
  int in_fmt;                  // InFmt of k, q, v (not float32: rotated-layout kernels only)
};

struct BwdArgs {
  const float* k;
  const float* v;
  const float* q;
  const float* d;
  const float* p;
  const float* r;
  const float* m0;
  const float* c0;
  const float* bm;
  const float* bc;
  const float* gy;
  const float* gmf;  // may be null (zero)
  const float* gcf;  // may be null (zero)
  float* gk;
  float* gv;
  float* gq;
  float* gd;   // null: not requested
  float* gp;   // null: not requested
  float* gr;   // null: not requested
  float* gm0;  // null: not requested
  float* gc0;  // null: not requested
  int64_t n;
  int64_t t;
  int64_t chunk;
  int64_t nb;
  float floor;
  int vec_kqd, vec_v, vec_pr;
  int rot4;  // D = 4 rotated-layout kernels allowed (see bssm_rot4.hip)
  int in_fmt;  // InFmt of k, q, v and gk, gq, gv (not float32: rotated-layout kernels only)
};

// Replay-history tensors of the saved-history ABI.
struct HistArgs {
  float* mp;  // [N,T,D,M] decay * mean before the token
  float* pp;  // [N,T,D,D] predicted covariance
  float* uh;  // [N,T,D]
  float* bh;  // [N,T]    1 / max(s, floor)
  float* eh;  // [N,T,M]
};

hipError_t launch_forward(int key_dim, bool fixed, const FwdArgs& a, hipStream_t stream);
hipError_t launch_backward(int key_dim, bool fixed, bool dynamics_grads, const BwdArgs& a, hipStream_t stream);
hipError_t launch_forward_saved(int key_dim, const FwdArgs& a, const HistArgs& h, hipStream_t stream);
hipError_t launch_backward_saved(int key_dim, bool dynamics_grads, const BwdArgs& a, const HistArgs& h,
                                 hipStream_t stream);
// D = 4, M = 8 kernels with the rotated per-lane layout (bssm_rot4.hip).
// Preconditions (checked by the C ABI, recorded in rot4): 16-byte aligned
// streams, T a positive multiple of 4, 8-byte aligned belief tensors, and for
// the backward a checkpoint chunk of kRot4Chunk tokens (a record per chunk)
// or 2 * kRot4Chunk (a record per 16-token tile; the tile's second chunk
// starts from the belief advanced on chip over its first 8 tokens).
constexpr int kRot4Chunk = 8;
hipError_t launch_forward_r4(bool fixed, const FwdArgs& a, hipStream_t stream);
hipError_t launch_backward_r4(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream);
// Row-per-sequence D = 4 kernels for small sequence counts (bssm_small.hip):
// used for float32 streams when the rotated-layout kernels apply and n is at
// most small_batch_limit(0) (forward) or small_batch_limit(1) (backward);
// as two / three waves per 4 sequences up to small_batch_limit(2) / (3).
hipError_t launch_forward_small(bool fixed, const FwdArgs& a, hipStream_t stream);
// The backward needs T a multiple of 16 and the kRot4Chunk checkpoint chunk.
hipError_t launch_backward_small(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream);
int64_t small_batch_limit(int direction);
int64_t set_small_batch_limit(int direction, int64_t limit);

// D = 1, M = 8 kernels with one lane per value column (bssm_d1.hip).  The
// forward needs 16-byte aligned streams, T and the checkpoint chunk
// multiples of 4; the backward also needs the checkpoint chunk to be 16 (the
// library's preferred one for D = 1) and T a positive multiple of 16.
// Other shapes take the generic kernels.
bool d1_forward_ok(const FwdArgs& a);
bool d1_backward_ok(const BwdArgs& a);
hipError_t launch_forward_d1(bool fixed, const FwdArgs& a, hipStream_t stream);
hipError_t launch_backward_d1(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream);

// D = 2, M = 8 kernels with two value columns per lane (bssm_d2.hip).  Both
// need 16-byte aligned streams and T a multiple of 4 (the forward takes any
// checkpoint chunk); the backward needs T > 0 and the checkpoint chunk 8
// (the library's preferred one for D = 2).
bool d2_forward_ok(const FwdArgs& a);
bool d2_backward_ok(const BwdArgs& a);
hipError_t launch_forward_d2(bool fixed, const FwdArgs& a, hipStream_t stream);
hipError_t launch_backward_d2(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream);

// D = 8, M = 8 kernels with 8 lanes per sequence in XOR order (bssm_d8.hip).
// The forward needs 16-byte aligned float32 streams and T a positive
// multiple of 8 (any checkpoint chunk); the checkpoint-replay backward also
// needs the checkpoint chunk 8 (the library's preferred one for D = 8) and
// 16-byte aligned checkpoint tensors.  Other shapes take the generic kernels.
bool d8_forward_ok(const FwdArgs& a);
hipError_t launch_forward_d8(bool fixed, const FwdArgs& a, hipStream_t stream);
bool d8_backward_ok(const BwdArgs& a);
hipError_t launch_backward_d8(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream);

// D = M = 64 kernels (bssm_d64.hip): one wave per sequence, lane = dimension.
// The backward replays each checkpoint chunk on chip before reversing a token,
// so its cost grows with the square of the chunk length; the autograd path
// checkpoints every kD64Checkpoint tokens.
constexpr int kD64Checkpoint = 8;
hipError_t launch_forward_d64(bool fixed, const FwdArgs& a, hipStream_t stream);
hipError_t launch_backward_d64(bool fixed, bool dyn, const BwdArgs& a, hipStream_t stream);

// Producer-fused D = 4, M = 8 layer core of the Bayes mixer (bssm_mixer.hip).
// Inputs are the bfloat16 projections in [B, T, *] layout, each with its own
// row stride (elements): queries, keys and decay logits [.., H * 4], values
// [.., H * 8], noise [.., H * 2] (process, observation per head).  The
// output and its gradient are float32 [B, T, H * 8]; the input gradients are
// contiguous, bfloat16 (float32 when grad_f32).  Belief tensors are the
// [B * H, ...] ones of the float32 ABI (sequence n = b * H + h).
struct MixArgs {
  const void *q, *k, *v, *dl, *nz;
  int64_t ldq, ldk, ldv, ldd, ldn;
  const float* m0;
  const float* c0;
  float* y;
  float* mT;
  float* cT;
  float* bm;
  float* bc;
  const float* bmr;  // backward: the forward's checkpoints
  const float* bcr;
  const float* gy;
  const float* gmf;  // may be null (zero)
  const float* gcf;  // may be null (zero)
  void *gq, *gk, *gv, *gdl, *gnz;  // gdl, gnz null: dynamics gradients not requested
  // Row strides (elements) of the gradient streams gq, gk, gv, gdl, gnz and
  // ggate; 0: contiguous rows of the stream's own width.
  int64_t ldgq, ldgk, ldgv, ldgd, ldgn, ldgg;
  float* gm0;  // may be null
  float* gc0;  // may be null
  int64_t b, t, h, chunk, nb;
  float floor;
  int grad_f32;
  // Readout epilogue (gated entry points; gate == nullptr: none).  Forward:
  // out = RMSNorm(bf16(read)) * norm_w * silu(gate), written bf16 (float32
  // when precise) [B, T, H * 8], and yb = bf16(read) [B, T, H * 8] saved for
  // the backward (y is not written).  Backward: gy is formed on chip from
  // gout (bf16 [B, T, H * 8]), yb and gate; ggate [B, T, H * 8] is written
  // bf16 (float32 when precise) and the weight gradient as per-wave partials
  // gw_part [B * H / 16, 8].
  const void* gate;
  int64_t ldg;
  const float* norm_w;
  float norm_eps;
  void* out;
  void* yb;
  const void* gout;
  void* ggate;
  float* gw_part;
  int precise;
  // Aux bias (bf16 [6 H]: decay logits 4 H, then noise 2 H; null: none),
  // added to the decay-logit and noise pieces in bf16 (one rounding) as
  // they are read.
  const void* abias;
};
hipError_t launch_mixer_forward(const MixArgs& a, hipStream_t stream);
hipError_t launch_mixer_backward(const MixArgs& a, hipStream_t stream);

// Rotation dynamics (bssm_rotation.hip): keys/queries [N, T, D], values,
// out, gy [N, T, 8], radii/angles/process (per pair) [N, T, D/2],
// observation [N, T]; belief tensors as the diagonal ABI.  vec: every stream
// 16-byte aligned with T a multiple of 4.
struct RotArgs {
  const float *k, *v, *q, *rad, *ang, *p, *r;
  const float *m0, *c0;
  float *y, *mT, *cT, *bm, *bc;
  const float *gy, *gmf, *gcf;
  float *gk, *gv, *gq, *grad, *gang, *gp, *gr, *gm0, *gc0;
  int64_t n, t, chunk, nb;
  float floor;
  int vec;
};
int rotation_checkpoint(int key_dim);
hipError_t launch_rotation_forward(int key_dim, const RotArgs& a, hipStream_t stream);
// Row-per-sequence rotation forward for D = 4, M = 8 (bssm_small.hip): used
// with 16-byte aligned streams (vec), T a multiple of 4 and 8-byte aligned
// mean tensors, for n up to small_batch_limit(4).
hipError_t launch_rotation_forward_small(const RotArgs& a, hipStream_t stream);
hipError_t launch_rotation_backward(int key_dim, const RotArgs& a, hipStream_t stream);

// Length-four causal depthwise filter on channels-last rows (bssm_conv4.hip):
// x [B, T, C] with row stride ldx (elements), y / gy / gx contiguous
// [B, T, C], weight float32 [C, 4], gw_part float32 [B, C, 4]; bfloat16 or
// float32 streams.
struct ConvArgs {
  const void* x;
  int64_t ldx;
  const float* w;
  void* y;
  const void* gy;
  void* gx;
  int64_t ldgx;  // row stride of gx (elements); 0: c
  float* gw_part;
  int64_t b, t, c;
  int bf16;
};
hipError_t launch_conv4_forward(const ConvArgs& a, hipStream_t stream);
hipError_t launch_conv4_backward(const ConvArgs& a, hipStream_t stream);
// The backward with the weight-gradient partials in the library's own device
// scratch (kConv4ScratchFloats floats per GPU) and their sum over the batch
// written to grad_weight [C, 4]; allocates nothing.  Needs b * c * 4 <=
// kConv4ScratchFloats (checked by the caller).
constexpr int64_t kConv4ScratchFloats = int64_t(1) << 21;
hipError_t launch_conv4_backward_noalloc(const ConvArgs& a, float* grad_weight, hipStream_t stream);
// Column sums over T of a bf16 [B, T, cols] view (row stride ld elements,
// cols and ld even, 4-byte aligned): out [B, cols] float32.
hipError_t launch_column_sums_bf16(const void* x, int64_t ld, int64_t b, int64_t t, int64_t cols, float* out,
                                  hipStream_t stream);
// Column sums of up to three row-major float32 matrices part[i] [rows[i],
// cols[i]] into out[i] [cols[i]], float32 or (bf16 != 0) bfloat16, in one
// launch (bssm_conv4.hip; `first` is filled by the launcher).
struct FoldArgs {
  const float* part[3];
  void* out[3];
  int64_t rows[3], cols[3], first[3];
  int count;
  int bf16;
};
hipError_t launch_fold(FoldArgs a, hipStream_t stream);

// One-pass (min, max, any non-finite) of up to kMaxStatTensors contiguous
// float32 / float64 tensors (bssm_checks.hip).  first_block[i] is the pass-1
// block where tensor i starts (prefix sums of stat_blocks(numel)); partials
// holds 3 * total_blocks floats, out 3 * count.
constexpr int kMaxStatTensors = 16;
struct StatArgs {
  const void* ptr[kMaxStatTensors];
  int64_t numel[kMaxStatTensors];
  int64_t first_block[kMaxStatTensors];
  int is_double[kMaxStatTensors];
  int count;
  int64_t total_blocks;
};
int64_t stat_blocks(int64_t numel);
hipError_t launch_value_stats(const StatArgs& a, float* partials, float* out, hipStream_t stream);

hipError_t launch_associative_scan(const float* k, const float* v, const float* q, const float* r,
                                   const float* m0, const float* c0, float* y, float* mT, float* cT,
                                   int64_t b, int64_t t, int d, int m, hipStream_t stream);
// Reverse of the scan for key dims up to kMaxBackwardD (value dims up to 64),
// T >= 1; ws holds b * t * (d * d + d * m) floats; gmT, gcT may be null.
constexpr int kMaxBackwardD = 16;
hipError_t launch_associative_scan_backward(const float* k, const float* v, const float* q, const float* r,
                                            const float* m0, const float* c0, const float* gy, const float* gmT,
                                            const float* gcT, float* ws, float* gk, float* gv, float* gq, float* gr,
                                            float* gm0, float* gc0, int64_t b, int64_t t, int d, int m,
                                            hipStream_t stream);

// Checkpoint interval at which the replay backward needs no in-chunk replay
// restarts (the register-history length for this key dimension).
int preferred_checkpoint(int key_dim);

}  // namespace bssm
