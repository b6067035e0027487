// C ABI of the gfx950 Bayesian-recurrence library (declared in include/bssm.h).
//
// The wrappers validate arguments, derive the checkpoint count and the
// 16-byte staging flags, and enqueue exactly one kernel per call on the
// caller's stream.  They never allocate, synchronise or keep state, which
// keeps every entry point usable under HIP graph capture.  Failures return a
// BSSM_ERR_* code and leave the message for bssm_last_error() on the calling
// thread (the reference raises through TORCH_CHECK,
// persistent_bayes_chunked_d4m8.cu:463-466, and checks launches with
// C10_CUDA_KERNEL_LAUNCH_CHECK, :467).

#include <cstdarg>
#include <cstdio>
#include <initializer_list>

#include "../../include/bssm.h"
#include "bssm_recurrence.h"

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_error[0] = '\0';
  return BSSM_OK;
}

bool supported(int d, int m) { return (m == 8 && (d == 1 || d == 2 || d == 4 || d == 8)) || (d == 64 && m == 64); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// The D = 4 rotated-layout kernels address each 16-sequence block through
// 32-bit buffer offsets, move every stream in 16-byte chunks and store the
// belief in 8-byte pieces.
bool rot4_ok(int d, int m, int64_t t, int64_t nb, bool streams16, std::initializer_list<const void*> belief) {
  if (d != 4 || m != 8 || t <= 0 || t % 4 != 0 || !streams16) return false;
  if ((nb + 1) * 128 * 16 >= ((int64_t)1 << 31)) return false;
  for (const void* p : belief)
    if (p != nullptr && !aligned8(p)) return false;
  return true;
}

// 16-byte staging is valid when every sequence row of the stream starts on a
// 16-byte boundary: base aligned and (T * width) a multiple of 4 floats.
int vec_flag(const float* p, int64_t t, int64_t width) {
  return (p == nullptr || aligned16(p)) && ((t * width) % 4 == 0);
}
// The same for a stream of the input format fmt (InFmt: 4, 8 or 16 elements per 16 bytes).
int vec_flag_fmt(const void* p, int64_t t, int64_t width, int fmt) {
  const int64_t per16 = fmt == bssm::kInF32 ? 4 : fmt == bssm::kInBf16 ? 8 : 16;
  return (p == nullptr || aligned16(p)) && ((t * width) % per16 == 0);
}
const char* fmt_name(int fmt) {
  return fmt == bssm::kInBf16 ? "bfloat16" : fmt == bssm::kInE4M3 ? "float8_e4m3fn" : "float8_e5m2";
}

int check_common(const char* fn, int d, int m, int64_t n, int64_t t, int64_t chunk, float floor) {
  if (!supported(d, m))
    return fail(BSSM_ERR_UNSUPPORTED, "%s: unsupported (key_dim, value_dim) = (%d, %d)", fn, d, m);
  if (n < 0 || t < 0) return fail(BSSM_ERR_ARGUMENT, "%s: negative size n=%lld t=%lld", fn, (long long)n, (long long)t);
  if (chunk <= 0) return fail(BSSM_ERR_ARGUMENT, "%s: chunk must be positive, got %lld", fn, (long long)chunk);
  if (!(floor > 0.f)) return fail(BSSM_ERR_ARGUMENT, "%s: denominator_floor must be positive", fn);
  if (n > (int64_t)0x7fffffff * 4) return fail(BSSM_ERR_ARGUMENT, "%s: n too large", fn);
  // Tile loads address up to 64 sequence rows with 32-bit lane offsets.
  if (t * (d > m ? d : m) > (int64_t)1 << 25)
    return fail(BSSM_ERR_ARGUMENT, "%s: t * max(key_dim, value_dim) must be <= 2^25, got t=%lld", fn, (long long)t);
  return BSSM_OK;
}

#define BSSM_REQUIRE(ptr)                                                          \
  do {                                                                             \
    if ((ptr) == nullptr && n > 0) return fail(BSSM_ERR_ARGUMENT, "%s: %s is null", fn, #ptr); \
  } while (0)

#define BSSM_REQUIRE_T(ptr)                                                                   \
  do {                                                                                        \
    if ((ptr) == nullptr && n > 0 && t > 0) return fail(BSSM_ERR_ARGUMENT, "%s: %s is null", fn, #ptr); \
  } while (0)

int launched(const char* fn, hipError_t err) {
  if (err != hipSuccess) return fail(BSSM_ERR_LAUNCH, "%s: kernel launch failed: %s", fn, hipGetErrorString(err));
  return ok();
}

// fmt (InFmt): keys, values and queries hold float32, bfloat16 or float8
// data (all but float32: rotated-layout kernels only; anything else is
// reported as unsupported).
int forward_impl(const char* fn, bool fixed, int d, int m, const float* keys, const float* values,
                 const float* queries, const float* decay, const float* process, const float* observation,
                 const float* mean0, const float* cov0, float* out, float* mean_final, float* cov_final,
                 float* bmean, float* bcov, int64_t n, int64_t t, int64_t chunk, float floor, void* stream,
                 int fmt = bssm::kInF32) {
  if (int rc = check_common(fn, d, m, n, t, chunk, floor)) return rc;
  BSSM_REQUIRE_T(keys);
  BSSM_REQUIRE_T(values);
  BSSM_REQUIRE_T(queries);
  BSSM_REQUIRE_T(out);
  if (!fixed) {
    BSSM_REQUIRE_T(decay);
    BSSM_REQUIRE_T(process);
    BSSM_REQUIRE_T(observation);
  }
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(mean_final);
  BSSM_REQUIRE(cov_final);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  bssm::FwdArgs a{};
  a.k = keys; a.v = values; a.q = queries; a.d = decay; a.p = process; a.r = observation;
  a.m0 = mean0; a.c0 = cov0; a.y = out; a.mT = mean_final; a.cT = cov_final; a.bm = bmean; a.bc = bcov;
  a.n = n; a.t = t; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = floor;
  a.in_fmt = fmt;
  a.vec_kqd = vec_flag_fmt(keys, t, d, fmt) && vec_flag_fmt(queries, t, d, fmt) && (fixed || vec_flag(decay, t, d));
  a.vec_v = vec_flag_fmt(values, t, m, fmt) && vec_flag(out, t, m);
  a.vec_pr = fixed || (vec_flag(process, t, 1) && vec_flag(observation, t, 1));
  a.rot4 = rot4_ok(d, m, t, a.nb, a.vec_kqd && a.vec_v && a.vec_pr, {mean0, cov0, mean_final, cov_final, bmean, bcov});
  if (fmt != bssm::kInF32 && !a.rot4 && n > 0)
    return fail(BSSM_ERR_UNSUPPORTED, "%s: %s inputs need D = 4, M = 8, T a positive multiple of 4 and "
                "16-byte aligned streams", fn, fmt_name(fmt));
  if (n == 0) return ok();
  return launched(fn, bssm::launch_forward(d, fixed, a, static_cast<hipStream_t>(stream)));
}

struct BwdOut {
  float *gk, *gv, *gq, *gd, *gp, *gr, *gm0, *gc0;
};

// fmt (InFmt): keys, values, queries and their gradients gk, gv, gq hold
// float32, bfloat16 or float8 data (all but float32: rotated-layout kernels
// only).
int backward_impl(const char* fn, bool fixed, bool dyn, int d, int m, const float* keys, const float* values,
                  const float* queries, const float* decay, const float* process, const float* observation,
                  const float* mean0, const float* cov0, const float* bmean, const float* bcov, const float* gy,
                  const float* gmf, const float* gcf, BwdOut o, int64_t n, int64_t t, int64_t chunk, float floor,
                  void* stream, int fmt = bssm::kInF32) {
  if (int rc = check_common(fn, d, m, n, t, chunk, floor)) return rc;
  BSSM_REQUIRE_T(keys);
  BSSM_REQUIRE_T(values);
  BSSM_REQUIRE_T(queries);
  BSSM_REQUIRE_T(gy);
  if (!fixed) {
    BSSM_REQUIRE_T(decay);
    BSSM_REQUIRE_T(process);
    BSSM_REQUIRE_T(observation);
  }
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  BSSM_REQUIRE_T(o.gk);
  BSSM_REQUIRE_T(o.gv);
  BSSM_REQUIRE_T(o.gq);
  bssm::BwdArgs a{};
  a.k = keys; a.v = values; a.q = queries; a.d = decay; a.p = process; a.r = observation;
  a.m0 = mean0; a.c0 = cov0; a.bm = bmean; a.bc = bcov; a.gy = gy; a.gmf = gmf; a.gcf = gcf;
  a.gk = o.gk; a.gv = o.gv; a.gq = o.gq; a.gd = o.gd; a.gp = o.gp; a.gr = o.gr; a.gm0 = o.gm0; a.gc0 = o.gc0;
  a.n = n; a.t = t; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = floor;
  a.in_fmt = fmt;
  a.vec_kqd = vec_flag_fmt(keys, t, d, fmt) && vec_flag_fmt(queries, t, d, fmt) && (fixed || vec_flag(decay, t, d)) &&
              vec_flag_fmt(o.gk, t, d, fmt) && vec_flag_fmt(o.gq, t, d, fmt) && vec_flag(o.gd, t, d);
  a.vec_v = vec_flag_fmt(values, t, m, fmt) && vec_flag(gy, t, m) && vec_flag_fmt(o.gv, t, m, fmt);
  a.vec_pr = (fixed || (vec_flag(process, t, 1) && vec_flag(observation, t, 1))) && vec_flag(o.gp, t, 1) &&
             vec_flag(o.gr, t, 1);
  a.rot4 = (chunk == bssm::kRot4Chunk || chunk == 2 * bssm::kRot4Chunk) &&
           rot4_ok(d, m, t, a.nb, a.vec_kqd && a.vec_v && a.vec_pr, {bmean, bcov, gmf, gcf, o.gm0, o.gc0});
  if (fmt != bssm::kInF32 && !a.rot4 && n > 0)
    return fail(BSSM_ERR_UNSUPPORTED, "%s: %s inputs need D = 4, M = 8, T a positive multiple of 4, "
                "checkpoint chunk %d or %d and 16-byte aligned streams", fn, fmt_name(fmt), bssm::kRot4Chunk,
                2 * bssm::kRot4Chunk);
  if (n == 0) return ok();
  return launched(fn, bssm::launch_backward(d, fixed, dyn, a, static_cast<hipStream_t>(stream)));
}

// Shape and layout checks of the producer-fused mixer entry points.  The
// kernels take 16 heads of one batch row per wave and address each batch
// row of a stream through a 32-bit buffer range of T rows.
int mixer_check(const char* fn, const void* const (&in)[5], const int64_t (&ld)[5], int64_t b, int64_t t, int64_t h,
                int64_t chunk, float floor) {
  static const int64_t kWidth[5] = {4, 4, 8, 4, 2};  // q, k, v, decay logits, noise (per head)
  static const char* kName[5] = {"q_proj", "k_proj", "v_proj", "decay_logits", "noise"};
  if (b < 0 || t < 0 || h < 0)
    return fail(BSSM_ERR_ARGUMENT, "%s: negative size b=%lld t=%lld h=%lld", fn, (long long)b, (long long)t,
                (long long)h);
  if (!(floor > 0.f)) return fail(BSSM_ERR_ARGUMENT, "%s: denominator_floor must be positive", fn);
  if (h % 16 != 0 || t <= 0 || t % 4 != 0 || chunk != bssm::kRot4Chunk)
    return fail(BSSM_ERR_UNSUPPORTED, "%s: needs heads %% 16 == 0, T a positive multiple of 4 and chunk == %d (got h=%lld t=%lld "
                "chunk=%lld)", fn, bssm::kRot4Chunk, (long long)h, (long long)t, (long long)chunk);
  if (b * h / 16 > 0x7fffffff) return fail(BSSM_ERR_ARGUMENT, "%s: batch * heads too large", fn);
  const int64_t nb = (t + chunk - 1) / chunk;
  if ((nb + 1) * 128 * 16 >= ((int64_t)1 << 31) || t * h * 32 >= ((int64_t)1 << 31))
    return fail(BSSM_ERR_ARGUMENT, "%s: T * heads too large for 32-bit stream offsets", fn);
  for (int i = 0; i < 5; ++i) {
    if (b * h * t > 0 && in[i] == nullptr) return fail(BSSM_ERR_ARGUMENT, "%s: %s is null", fn, kName[i]);
    if (ld[i] < kWidth[i] * h || ld[i] % 8 != 0 || !aligned16(in[i]))
      return fail(BSSM_ERR_UNSUPPORTED, "%s: %s needs a row stride >= %lld elements, a multiple of 8, and a "
                  "16-byte aligned base (got ld=%lld)", fn, kName[i], (long long)(kWidth[i] * h), (long long)ld[i]);
    if ((t + 16) * ld[i] * 2 >= ((int64_t)1 << 31))
      return fail(BSSM_ERR_ARGUMENT, "%s: T * ld of %s too large for 32-bit stream offsets", fn, kName[i]);
  }
  return BSSM_OK;
}

// Checks of the readout-epilogue streams (gate view; contiguous [B, T, H * 8] tensors).
int epilogue_check(const char* fn, const void* gate, int64_t ldg, const float* norm_weight, float norm_eps,
                   std::initializer_list<const void*> contiguous, int64_t b, int64_t t, int64_t h) {
  if (b * h * t > 0 && (gate == nullptr || norm_weight == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: gate and norm_weight are required", fn);
  if (ldg < 8 * h || ldg % 8 != 0 || !aligned16(gate))
    return fail(BSSM_ERR_UNSUPPORTED, "%s: gate needs a row stride >= %lld elements, a multiple of 8, and a 16-byte "
                "aligned base (got ld=%lld)", fn, (long long)(8 * h), (long long)ldg);
  if ((t + 16) * ldg * 2 >= ((int64_t)1 << 31))
    return fail(BSSM_ERR_ARGUMENT, "%s: T * ld of gate too large for 32-bit stream offsets", fn);
  if (!(norm_eps >= 0.f)) return fail(BSSM_ERR_ARGUMENT, "%s: norm_eps must be non-negative", fn);
  for (const void* p : contiguous)
    if (b * h * t > 0 && (p == nullptr || !aligned16(p)))
      return fail(BSSM_ERR_ARGUMENT, "%s: epilogue tensors must be non-null and 16-byte aligned", fn);
  return BSSM_OK;
}

int conv_check(const char* fn, int bf16, const void* x, int64_t ldx, const float* weight,
               std::initializer_list<const void*> contiguous, int64_t b, int64_t t, int64_t c) {
  const int64_t n = bf16 ? 8 : 4, elem = bf16 ? 2 : 4;
  if (b < 0 || t < 0 || c < 0) return fail(BSSM_ERR_ARGUMENT, "%s: negative size", fn);
  if (c % n != 0 || ldx < c || ldx % n != 0)
    return fail(BSSM_ERR_UNSUPPORTED, "%s: channels and the row stride must be multiples of %lld (16 bytes), "
                "row stride >= channels (got c=%lld ldx=%lld)", fn, (long long)n, (long long)c, (long long)ldx);
  if ((t + 16) * ldx * elem >= ((int64_t)1 << 31) || (t + 16) * c * elem >= ((int64_t)1 << 31))
    return fail(BSSM_ERR_ARGUMENT, "%s: T * row bytes too large for 32-bit stream offsets", fn);
  if (b * ((c / n + 63) / 64) > 0x7fffffff) return fail(BSSM_ERR_ARGUMENT, "%s: batch * channels too large", fn);
  if (b * t * c == 0) return BSSM_OK;
  if (x == nullptr || weight == nullptr) return fail(BSSM_ERR_ARGUMENT, "%s: x and weight are required", fn);
  if (!aligned16(x) || !aligned16(weight)) return fail(BSSM_ERR_ARGUMENT, "%s: x and weight must be 16-byte aligned", fn);
  for (const void* p : contiguous)
    if (p == nullptr || !aligned16(p)) return fail(BSSM_ERR_ARGUMENT, "%s: outputs must be non-null, 16-byte aligned", fn);
  return BSSM_OK;
}

}  // namespace

extern "C" {

const char* bssm_last_error(void) { return g_error; }

int bssm_abi_version(void) { return 9; }

int bssm_supported(int key_dim, int value_dim) { return supported(key_dim, value_dim) ? 1 : 0; }

int bssm_preferred_checkpoint(int key_dim) { return bssm::preferred_checkpoint(key_dim); }

int bssm_forward_chunked(int key_dim, int value_dim, const float* keys, const float* values, const float* queries,
                         const float* decay, const float* process, const float* observation, const float* mean0,
                         const float* cov0, float* out, float* mean_final, float* cov_final, float* bmean,
                         float* bcov, int64_t n, int64_t t, int64_t chunk, float denominator_floor, void* stream) {
  return forward_impl("bssm_forward_chunked", false, key_dim, value_dim, keys, values, queries, decay, process,
                      observation, mean0, cov0, out, mean_final, cov_final, bmean, bcov, n, t, chunk,
                      denominator_floor, stream);
}

int bssm_forward_chunked_fixed(int key_dim, int value_dim, const float* keys, const float* values,
                               const float* queries, const float* decay, const float* process,
                               const float* observation, const float* mean0, const float* cov0, float* out,
                               float* mean_final, float* cov_final, float* bmean, float* bcov, int64_t n, int64_t t,
                               int64_t chunk, float denominator_floor, void* stream) {
  return forward_impl("bssm_forward_chunked_fixed", true, key_dim, value_dim, keys, values, queries, decay, process,
                      observation, mean0, cov0, out, mean_final, cov_final, bmean, bcov, n, t, chunk,
                      denominator_floor, stream);
}

int bssm_backward_chunked(int key_dim, int value_dim, const float* keys, const float* values, const float* queries,
                          const float* decay, const float* process, const float* observation, const float* mean0,
                          const float* cov0, const float* bmean, const float* bcov, const float* gy,
                          const float* gmf, const float* gcf, float* gk, float* gv, float* gq, float* gd, float* gp,
                          float* gr, float* gm0, float* gc0, int64_t n, int64_t t, int64_t chunk,
                          float denominator_floor, void* stream) {
  const char* fn = "bssm_backward_chunked";
  if (n > 0 && (gm0 == nullptr || gc0 == nullptr || (t > 0 && (gd == nullptr || gp == nullptr || gr == nullptr))))
    return fail(BSSM_ERR_ARGUMENT, "%s: all eight gradient outputs are required", fn);
  return backward_impl(fn, false, true, key_dim, value_dim, keys, values, queries, decay, process, observation,
                       mean0, cov0, bmean, bcov, gy, gmf, gcf, BwdOut{gk, gv, gq, gd, gp, gr, gm0, gc0}, n, t,
                       chunk, denominator_floor, stream);
}

int bssm_backward_chunked_lean(int key_dim, int value_dim, const float* keys, const float* values,
                               const float* queries, const float* decay, const float* process,
                               const float* observation, const float* mean0, const float* cov0, const float* bmean,
                               const float* bcov, const float* gy, const float* gmf, const float* gcf, float* gk,
                               float* gv, float* gq, int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                               void* stream) {
  return backward_impl("bssm_backward_chunked_lean", false, false, key_dim, value_dim, keys, values, queries, decay,
                       process, observation, mean0, cov0, bmean, bcov, gy, gmf, gcf,
                       BwdOut{gk, gv, gq, nullptr, nullptr, nullptr, nullptr, nullptr}, n, t, chunk,
                       denominator_floor, stream);
}

int bssm_backward_chunked_noinitial(int key_dim, int value_dim, const float* keys, const float* values,
                                    const float* queries, const float* decay, const float* process,
                                    const float* observation, const float* mean0, const float* cov0,
                                    const float* bmean, const float* bcov, const float* gy, const float* gmf,
                                    const float* gcf, float* gk, float* gv, float* gq, float* gd, float* gp,
                                    float* gr, int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                    void* stream) {
  const char* fn = "bssm_backward_chunked_noinitial";
  if (n > 0 && t > 0 && (gd == nullptr || gp == nullptr || gr == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: gd, gp and gr are required", fn);
  return backward_impl(fn, false, true, key_dim, value_dim, keys, values, queries, decay, process, observation,
                       mean0, cov0, bmean, bcov, gy, gmf, gcf, BwdOut{gk, gv, gq, gd, gp, gr, nullptr, nullptr}, n,
                       t, chunk, denominator_floor, stream);
}

int bssm_backward_chunked_fixed(int key_dim, int value_dim, const float* keys, const float* values,
                                const float* queries, const float* decay, const float* process,
                                const float* observation, const float* mean0, const float* cov0, const float* bmean,
                                const float* bcov, const float* gy, const float* gmf, const float* gcf, float* gk,
                                float* gv, float* gq, float* gd, float* gp, float* gr, float* gm0, float* gc0,
                                int64_t n, int64_t t, int64_t chunk, float denominator_floor, void* stream) {
  const char* fn = "bssm_backward_chunked_fixed";
  if (n > 0 && (gm0 == nullptr || gc0 == nullptr || (t > 0 && (gd == nullptr || gp == nullptr || gr == nullptr))))
    return fail(BSSM_ERR_ARGUMENT, "%s: all eight gradient outputs are required", fn);
  return backward_impl(fn, true, false, key_dim, value_dim, keys, values, queries, decay, process, observation,
                       mean0, cov0, bmean, bcov, gy, gmf, gcf, BwdOut{gk, gv, gq, gd, gp, gr, gm0, gc0}, n, t,
                       chunk, denominator_floor, stream);
}

int bssm_backward_chunked_lean_fixed(int key_dim, int value_dim, const float* keys, const float* values,
                                     const float* queries, const float* decay, const float* process,
                                     const float* observation, const float* mean0, const float* cov0,
                                     const float* bmean, const float* bcov, const float* gy, const float* gmf,
                                     const float* gcf, float* gk, float* gv, float* gq, int64_t n, int64_t t,
                                     int64_t chunk, float denominator_floor, void* stream) {
  return backward_impl("bssm_backward_chunked_lean_fixed", true, false, key_dim, value_dim, keys, values, queries,
                       decay, process, observation, mean0, cov0, bmean, bcov, gy, gmf, gcf,
                       BwdOut{gk, gv, gq, nullptr, nullptr, nullptr, nullptr, nullptr}, n, t, chunk,
                       denominator_floor, stream);
}

int bssm_backward_chunked_noinitial_fixed(int key_dim, int value_dim, const float* keys, const float* values,
                                          const float* queries, const float* decay, const float* process,
                                          const float* observation, const float* mean0, const float* cov0,
                                          const float* bmean, const float* bcov, const float* gy, const float* gmf,
                                          const float* gcf, float* gk, float* gv, float* gq, float* gd, float* gp,
                                          float* gr, int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                          void* stream) {
  const char* fn = "bssm_backward_chunked_noinitial_fixed";
  if (n > 0 && t > 0 && (gd == nullptr || gp == nullptr || gr == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: gd, gp and gr are required", fn);
  return backward_impl(fn, true, false, key_dim, value_dim, keys, values, queries, decay, process, observation,
                       mean0, cov0, bmean, bcov, gy, gmf, gcf, BwdOut{gk, gv, gq, gd, gp, gr, nullptr, nullptr}, n,
                       t, chunk, denominator_floor, stream);
}

int bssm_forward_chunked_saved(int key_dim, int value_dim, const float* keys, const float* values,
                               const float* queries, const float* decay, const float* process,
                               const float* observation, const float* mean0, const float* cov0, float* out,
                               float* mean_final, float* cov_final, float* bmean, float* bcov, float* mp, float* pp,
                               float* uh, float* bh, float* eh, int64_t n, int64_t t, int64_t chunk,
                               float denominator_floor, void* stream) {
  const char* fn = "bssm_forward_chunked_saved";
  if (int rc = check_common(fn, key_dim, value_dim, n, t, chunk, denominator_floor)) return rc;
  if (chunk != t) return fail(BSSM_ERR_ARGUMENT, "%s: saved history requires one full-sequence chunk", fn);
  BSSM_REQUIRE_T(mp);
  BSSM_REQUIRE_T(pp);
  BSSM_REQUIRE_T(uh);
  BSSM_REQUIRE_T(bh);
  BSSM_REQUIRE_T(eh);
  BSSM_REQUIRE_T(keys);
  BSSM_REQUIRE_T(values);
  BSSM_REQUIRE_T(queries);
  BSSM_REQUIRE_T(decay);
  BSSM_REQUIRE_T(process);
  BSSM_REQUIRE_T(observation);
  BSSM_REQUIRE_T(out);
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(mean_final);
  BSSM_REQUIRE(cov_final);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  bssm::FwdArgs a{};
  a.k = keys; a.v = values; a.q = queries; a.d = decay; a.p = process; a.r = observation;
  a.m0 = mean0; a.c0 = cov0; a.y = out; a.mT = mean_final; a.cT = cov_final; a.bm = bmean; a.bc = bcov;
  a.n = n; a.t = t; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = denominator_floor;
  bssm::HistArgs h{mp, pp, uh, bh, eh};
  if (n == 0) return ok();
  return launched(fn, bssm::launch_forward_saved(key_dim, a, h, static_cast<hipStream_t>(stream)));
}

static int backward_saved_impl(const char* fn, bool dyn, int key_dim, int value_dim, const float* keys,
                               const float* values, const float* queries, const float* decay, const float* process,
                               const float* observation, const float* mean0, const float* cov0, const float* bmean,
                               const float* bcov, const float* mp, const float* pp, const float* uh, const float* bh,
                               const float* eh, const float* gy, const float* gmf, const float* gcf, BwdOut o,
                               int64_t n, int64_t t, int64_t chunk, float floor, void* stream) {
  if (int rc = check_common(fn, key_dim, value_dim, n, t, chunk, floor)) return rc;
  if (chunk != t) return fail(BSSM_ERR_ARGUMENT, "%s: saved history requires one full-sequence chunk", fn);
  BSSM_REQUIRE_T(mp);
  BSSM_REQUIRE_T(pp);
  BSSM_REQUIRE_T(uh);
  BSSM_REQUIRE_T(bh);
  BSSM_REQUIRE_T(eh);
  BSSM_REQUIRE_T(keys);
  BSSM_REQUIRE_T(queries);
  BSSM_REQUIRE_T(decay);
  BSSM_REQUIRE_T(process);
  BSSM_REQUIRE_T(observation);
  BSSM_REQUIRE_T(gy);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  BSSM_REQUIRE_T(o.gk);
  BSSM_REQUIRE_T(o.gv);
  BSSM_REQUIRE_T(o.gq);
  bssm::BwdArgs a{};
  a.k = keys; a.v = values; a.q = queries; a.d = decay; a.p = process; a.r = observation;
  a.m0 = mean0; a.c0 = cov0; a.bm = bmean; a.bc = bcov; a.gy = gy; a.gmf = gmf; a.gcf = gcf;
  a.gk = o.gk; a.gv = o.gv; a.gq = o.gq; a.gd = o.gd; a.gp = o.gp; a.gr = o.gr; a.gm0 = o.gm0; a.gc0 = o.gc0;
  a.n = n; a.t = t; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = floor;
  bssm::HistArgs h{const_cast<float*>(mp), const_cast<float*>(pp), const_cast<float*>(uh), const_cast<float*>(bh),
                   const_cast<float*>(eh)};
  if (n == 0) return ok();
  return launched(fn, bssm::launch_backward_saved(key_dim, dyn, a, h, static_cast<hipStream_t>(stream)));
}

int bssm_backward_chunked_saved(int key_dim, int value_dim, const float* keys, const float* values,
                                const float* queries, const float* decay, const float* process,
                                const float* observation, const float* mean0, const float* cov0, const float* bmean,
                                const float* bcov, const float* mp, const float* pp, const float* uh, const float* bh,
                                const float* eh, const float* gy, const float* gmf, const float* gcf, float* gk,
                                float* gv, float* gq, float* gd, float* gp, float* gr, float* gm0, float* gc0,
                                int64_t n, int64_t t, int64_t chunk, float denominator_floor, void* stream) {
  const char* fn = "bssm_backward_chunked_saved";
  if (n > 0 && (gm0 == nullptr || gc0 == nullptr || (t > 0 && (gd == nullptr || gp == nullptr || gr == nullptr))))
    return fail(BSSM_ERR_ARGUMENT, "%s: all eight gradient outputs are required", fn);
  return backward_saved_impl(fn, true, key_dim, value_dim, keys, values, queries, decay, process, observation, mean0,
                             cov0, bmean, bcov, mp, pp, uh, bh, eh, gy, gmf, gcf,
                             BwdOut{gk, gv, gq, gd, gp, gr, gm0, gc0}, n, t, chunk, denominator_floor, stream);
}

int bssm_backward_chunked_saved_lean(int key_dim, int value_dim, const float* keys, const float* values,
                                     const float* queries, const float* decay, const float* process,
                                     const float* observation, const float* mean0, const float* cov0,
                                     const float* bmean, const float* bcov, const float* mp, const float* pp,
                                     const float* uh, const float* bh, const float* eh, const float* gy,
                                     const float* gmf, const float* gcf, float* gk, float* gv, float* gq, int64_t n,
                                     int64_t t, int64_t chunk, float denominator_floor, void* stream) {
  return backward_saved_impl("bssm_backward_chunked_saved_lean", false, key_dim, value_dim, keys, values, queries,
                             decay, process, observation, mean0, cov0, bmean, bcov, mp, pp, uh, bh, eh, gy, gmf, gcf,
                             BwdOut{gk, gv, gq, nullptr, nullptr, nullptr, nullptr, nullptr}, n, t, chunk,
                             denominator_floor, stream);
}

int bssm_forward_chunked_bf16(int key_dim, int value_dim, int fixed, const void* keys, const void* values,
                              const void* queries, const float* decay, const float* process,
                              const float* observation, const float* mean0, const float* cov0, float* out,
                              float* mean_final, float* cov_final, float* bmean, float* bcov, int64_t n, int64_t t,
                              int64_t chunk, float denominator_floor, void* stream) {
  return forward_impl("bssm_forward_chunked_bf16", fixed != 0, key_dim, value_dim, static_cast<const float*>(keys),
                      static_cast<const float*>(values), static_cast<const float*>(queries), decay, process,
                      observation, mean0, cov0, out, mean_final, cov_final, bmean, bcov, n, t, chunk,
                      denominator_floor, stream, bssm::kInBf16);
}

int bssm_backward_chunked_bf16(int key_dim, int value_dim, int fixed, const void* keys, const void* values,
                               const void* queries, const float* decay, const float* process,
                               const float* observation, const float* mean0, const float* cov0, const float* bmean,
                               const float* bcov, const float* gy, const float* gmf, const float* gcf, void* gk,
                               void* gv, void* gq, float* gd, float* gp, float* gr, float* gm0, float* gc0,
                               int64_t n, int64_t t, int64_t chunk, float denominator_floor, void* stream) {
  const char* fn = "bssm_backward_chunked_bf16";
  const bool dyn = gd != nullptr;
  if ((gd == nullptr) != (gp == nullptr) || (gd == nullptr) != (gr == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: gd, gp and gr must be given together or all be null", fn);
  return backward_impl(fn, fixed != 0, dyn && !fixed, key_dim, value_dim, static_cast<const float*>(keys),
                       static_cast<const float*>(values), static_cast<const float*>(queries), decay, process,
                       observation, mean0, cov0, bmean, bcov, gy, gmf, gcf,
                       BwdOut{static_cast<float*>(gk), static_cast<float*>(gv), static_cast<float*>(gq), gd, gp, gr,
                              gm0, gc0},
                       n, t, chunk, denominator_floor, stream, bssm::kInBf16);
}

int bssm_forward_chunked_fp8(int key_dim, int value_dim, int fixed, int format, const void* keys,
                             const void* values, const void* queries, const float* decay, const float* process,
                             const float* observation, const float* mean0, const float* cov0, float* out,
                             float* mean_final, float* cov_final, float* bmean, float* bcov, int64_t n, int64_t t,
                             int64_t chunk, float denominator_floor, void* stream) {
  const char* fn = "bssm_forward_chunked_fp8";
  if (format != 0 && format != 1)
    return fail(BSSM_ERR_ARGUMENT, "%s: format must be 0 (float8_e4m3fn) or 1 (float8_e5m2), got %d", fn, format);
  return forward_impl(fn, fixed != 0, key_dim, value_dim, static_cast<const float*>(keys),
                      static_cast<const float*>(values), static_cast<const float*>(queries), decay, process,
                      observation, mean0, cov0, out, mean_final, cov_final, bmean, bcov, n, t, chunk,
                      denominator_floor, stream, format == 0 ? bssm::kInE4M3 : bssm::kInE5M2);
}

int bssm_backward_chunked_fp8(int key_dim, int value_dim, int fixed, int format, const void* keys,
                              const void* values, const void* queries, const float* decay, const float* process,
                              const float* observation, const float* mean0, const float* cov0, const float* bmean,
                              const float* bcov, const float* gy, const float* gmf, const float* gcf, void* gk,
                              void* gv, void* gq, float* gd, float* gp, float* gr, float* gm0, float* gc0,
                              int64_t n, int64_t t, int64_t chunk, float denominator_floor, void* stream) {
  const char* fn = "bssm_backward_chunked_fp8";
  if (format != 0 && format != 1)
    return fail(BSSM_ERR_ARGUMENT, "%s: format must be 0 (float8_e4m3fn) or 1 (float8_e5m2), got %d", fn, format);
  const bool dyn = gd != nullptr;
  if ((gd == nullptr) != (gp == nullptr) || (gd == nullptr) != (gr == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: gd, gp and gr must be given together or all be null", fn);
  return backward_impl(fn, fixed != 0, dyn && !fixed, key_dim, value_dim, static_cast<const float*>(keys),
                       static_cast<const float*>(values), static_cast<const float*>(queries), decay, process,
                       observation, mean0, cov0, bmean, bcov, gy, gmf, gcf,
                       BwdOut{static_cast<float*>(gk), static_cast<float*>(gv), static_cast<float*>(gq), gd, gp, gr,
                              gm0, gc0},
                       n, t, chunk, denominator_floor, stream, format == 0 ? bssm::kInE4M3 : bssm::kInE5M2);
}

int64_t bssm_value_stats_workspace(int count, const int64_t* numels) {
  if (count < 0 || count > bssm::kMaxStatTensors || (count > 0 && numels == nullptr)) return -1;
  int64_t blocks = 0;
  for (int i = 0; i < count; ++i) {
    if (numels[i] < 0) return -1;
    blocks += bssm::stat_blocks(numels[i]);
  }
  return 3 * blocks;
}

int bssm_value_stats(int count, const void* const* tensors, const int64_t* numels, const int* is_double,
                     float* workspace, int64_t workspace_floats, float* out, void* stream) {
  const char* fn = "bssm_value_stats";
  if (count < 0 || count > bssm::kMaxStatTensors)
    return fail(BSSM_ERR_ARGUMENT, "%s: count must be in [0, %d], got %d", fn, bssm::kMaxStatTensors, count);
  if (count == 0) return ok();
  if (tensors == nullptr || numels == nullptr || is_double == nullptr || out == nullptr)
    return fail(BSSM_ERR_ARGUMENT, "%s: tensors, numels, is_double and out are required", fn);
  bssm::StatArgs a{};
  a.count = count;
  int64_t blocks = 0;
  for (int i = 0; i < count; ++i) {
    if (numels[i] < 0) return fail(BSSM_ERR_ARGUMENT, "%s: negative numel", fn);
    if (numels[i] > 0 && tensors[i] == nullptr) return fail(BSSM_ERR_ARGUMENT, "%s: tensor %d is null", fn, i);
    a.ptr[i] = tensors[i];
    a.numel[i] = numels[i];
    a.is_double[i] = is_double[i] != 0;
    a.first_block[i] = blocks;
    blocks += bssm::stat_blocks(numels[i]);
  }
  a.total_blocks = blocks;
  if (blocks > 0x7fffffff) return fail(BSSM_ERR_ARGUMENT, "%s: tensors too large", fn);
  if (workspace_floats < 3 * blocks || (blocks > 0 && workspace == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: workspace needs %lld floats", fn, (long long)(3 * blocks));
  return launched(fn, bssm::launch_value_stats(a, workspace, out, static_cast<hipStream_t>(stream)));
}

int bssm_round_float8(int format, const float* x, uint8_t* out, int64_t count) {
  const char* fn = "bssm_round_float8";
  if (format != 0 && format != 1)
    return fail(BSSM_ERR_ARGUMENT, "%s: format must be 0 (float8_e4m3fn) or 1 (float8_e5m2), got %d", fn, format);
  if (count < 0 || (count > 0 && (x == nullptr || out == nullptr)))
    return fail(BSSM_ERR_ARGUMENT, "%s: needs count >= 0 and non-null arrays", fn);
  for (int64_t i = 0; i < count; ++i)
    out[i] = static_cast<uint8_t>(format == 0 ? bssm::float_to_f8<bssm::kInE4M3>(x[i])
                                              : bssm::float_to_f8<bssm::kInE5M2>(x[i]));
  return ok();
}

int bssm_mixer_forward(const void* q_proj, int64_t ldq, const void* k_proj, int64_t ldk, const void* v_proj,
                       int64_t ldv, const void* decay_logits, int64_t ldd, const void* noise, int64_t ldn,
                       const float* mean0, const float* cov0, float* read, float* mean_final, float* cov_final,
                       float* bmean, float* bcov, int64_t batch, int64_t t, int64_t heads, int64_t chunk,
                       float denominator_floor, void* stream) {
  const char* fn = "bssm_mixer_forward";
  if (int rc = mixer_check(fn, {q_proj, k_proj, v_proj, decay_logits, noise}, {ldq, ldk, ldv, ldd, ldn}, batch, t,
                           heads, chunk, denominator_floor))
    return rc;
  const int64_t n = batch * heads;
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(mean_final);
  BSSM_REQUIRE(cov_final);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  BSSM_REQUIRE_T(read);
  for (const void* p : {(const void*)mean0, (const void*)cov0, (const void*)mean_final, (const void*)cov_final,
                        (const void*)bmean, (const void*)bcov})
    if (p != nullptr && !aligned8(p)) return fail(BSSM_ERR_ARGUMENT, "%s: belief tensors must be 8-byte aligned", fn);
  if (read != nullptr && !aligned16(read)) return fail(BSSM_ERR_ARGUMENT, "%s: read must be 16-byte aligned", fn);
  bssm::MixArgs a{};
  a.q = q_proj; a.k = k_proj; a.v = v_proj; a.dl = decay_logits; a.nz = noise;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldd = ldd; a.ldn = ldn;
  a.m0 = mean0; a.c0 = cov0; a.y = read; a.mT = mean_final; a.cT = cov_final; a.bm = bmean; a.bc = bcov;
  a.b = batch; a.t = t; a.h = heads; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = denominator_floor;
  if (n == 0) return ok();
  return launched(fn, bssm::launch_mixer_forward(a, static_cast<hipStream_t>(stream)));
}

int bssm_mixer_backward(const void* q_proj, int64_t ldq, const void* k_proj, int64_t ldk, const void* v_proj,
                        int64_t ldv, const void* decay_logits, int64_t ldd, const void* noise, int64_t ldn,
                        const float* mean0, const float* cov0, const float* bmean, const float* bcov,
                        const float* grad_read, const float* gmf, const float* gcf, void* grad_q, void* grad_k,
                        void* grad_v, void* grad_decay_logits, void* grad_noise, float* gm0, float* gc0,
                        int64_t batch, int64_t t, int64_t heads, int64_t chunk, float denominator_floor,
                        int grad_f32, void* stream) {
  const char* fn = "bssm_mixer_backward";
  if (int rc = mixer_check(fn, {q_proj, k_proj, v_proj, decay_logits, noise}, {ldq, ldk, ldv, ldd, ldn}, batch, t,
                           heads, chunk, denominator_floor))
    return rc;
  const int64_t n = batch * heads;
  if ((grad_decay_logits == nullptr) != (grad_noise == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: grad_decay_logits and grad_noise must be given together or both be null", fn);
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  BSSM_REQUIRE_T(grad_read);
  BSSM_REQUIRE_T(grad_q);
  BSSM_REQUIRE_T(grad_k);
  BSSM_REQUIRE_T(grad_v);
  for (const void* p : {(const void*)bmean, (const void*)bcov, (const void*)gmf, (const void*)gcf, (const void*)gm0,
                        (const void*)gc0})
    if (p != nullptr && !aligned8(p)) return fail(BSSM_ERR_ARGUMENT, "%s: belief tensors must be 8-byte aligned", fn);
  for (const void* p : {(const void*)grad_read, (const void*)grad_q, (const void*)grad_k, (const void*)grad_v,
                        (const void*)grad_decay_logits, (const void*)grad_noise})
    if (p != nullptr && !aligned16(p))
      return fail(BSSM_ERR_ARGUMENT, "%s: grad_read and the projection gradients must be 16-byte aligned", fn);
  bssm::MixArgs a{};
  a.q = q_proj; a.k = k_proj; a.v = v_proj; a.dl = decay_logits; a.nz = noise;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldd = ldd; a.ldn = ldn;
  a.m0 = mean0; a.c0 = cov0; a.bmr = bmean; a.bcr = bcov; a.gy = grad_read; a.gmf = gmf; a.gcf = gcf;
  a.gq = grad_q; a.gk = grad_k; a.gv = grad_v; a.gdl = grad_decay_logits; a.gnz = grad_noise;
  a.gm0 = gm0; a.gc0 = gc0;
  a.b = batch; a.t = t; a.h = heads; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = denominator_floor;
  a.grad_f32 = grad_f32 != 0;
  if (n == 0) return ok();
  return launched(fn, bssm::launch_mixer_backward(a, static_cast<hipStream_t>(stream)));
}

int bssm_mixer_gated_forward(const void* q_proj, int64_t ldq, const void* k_proj, int64_t ldk, const void* v_proj,
                             int64_t ldv, const void* decay_logits, int64_t ldd, const void* noise, int64_t ldn,
                             const void* gate, int64_t ldg, const float* norm_weight, float norm_eps,
                             const float* mean0, const float* cov0, void* out, void* read_bf16, float* mean_final,
                             float* cov_final, float* bmean, float* bcov, int64_t batch, int64_t t, int64_t heads,
                             int64_t chunk, float denominator_floor, int precise, void* stream) {
  const char* fn = "bssm_mixer_gated_forward";
  if (int rc = mixer_check(fn, {q_proj, k_proj, v_proj, decay_logits, noise}, {ldq, ldk, ldv, ldd, ldn}, batch, t,
                           heads, chunk, denominator_floor))
    return rc;
  if (int rc = epilogue_check(fn, gate, ldg, norm_weight, norm_eps, {out, read_bf16}, batch, t, heads)) return rc;
  const int64_t n = batch * heads;
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(mean_final);
  BSSM_REQUIRE(cov_final);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  for (const void* p : {(const void*)mean0, (const void*)cov0, (const void*)mean_final, (const void*)cov_final,
                        (const void*)bmean, (const void*)bcov})
    if (p != nullptr && !aligned8(p)) return fail(BSSM_ERR_ARGUMENT, "%s: belief tensors must be 8-byte aligned", fn);
  bssm::MixArgs a{};
  a.q = q_proj; a.k = k_proj; a.v = v_proj; a.dl = decay_logits; a.nz = noise;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldd = ldd; a.ldn = ldn;
  a.m0 = mean0; a.c0 = cov0; a.mT = mean_final; a.cT = cov_final; a.bm = bmean; a.bc = bcov;
  a.gate = gate; a.ldg = ldg; a.norm_w = norm_weight; a.norm_eps = norm_eps; a.out = out; a.yb = read_bf16;
  a.precise = precise != 0;
  a.b = batch; a.t = t; a.h = heads; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = denominator_floor;
  if (n == 0) return ok();
  return launched(fn, bssm::launch_mixer_forward(a, static_cast<hipStream_t>(stream)));
}

int bssm_mixer_gated_backward(const void* q_proj, int64_t ldq, const void* k_proj, int64_t ldk, const void* v_proj,
                              int64_t ldv, const void* decay_logits, int64_t ldd, const void* noise, int64_t ldn,
                              const void* gate, int64_t ldg, const float* norm_weight, float norm_eps,
                              const float* mean0, const float* cov0, const float* bmean, const float* bcov,
                              const void* read_bf16, const void* grad_out, const float* gmf, const float* gcf,
                              void* grad_q, void* grad_k, void* grad_v, void* grad_decay_logits, void* grad_noise,
                              void* grad_gate, float* grad_norm_weight_partials, float* gm0, float* gc0,
                              int64_t batch, int64_t t, int64_t heads, int64_t chunk, float denominator_floor,
                              int precise, void* stream) {
  const char* fn = "bssm_mixer_gated_backward";
  if (int rc = mixer_check(fn, {q_proj, k_proj, v_proj, decay_logits, noise}, {ldq, ldk, ldv, ldd, ldn}, batch, t,
                           heads, chunk, denominator_floor))
    return rc;
  if (int rc = epilogue_check(fn, gate, ldg, norm_weight, norm_eps,
                              {read_bf16, grad_out, grad_gate, grad_norm_weight_partials}, batch, t, heads))
    return rc;
  const int64_t n = batch * heads;
  if ((grad_decay_logits == nullptr) != (grad_noise == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: grad_decay_logits and grad_noise must be given together or both be null", fn);
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  BSSM_REQUIRE_T(grad_q);
  BSSM_REQUIRE_T(grad_k);
  BSSM_REQUIRE_T(grad_v);
  for (const void* p : {(const void*)bmean, (const void*)bcov, (const void*)gmf, (const void*)gcf, (const void*)gm0,
                        (const void*)gc0})
    if (p != nullptr && !aligned8(p)) return fail(BSSM_ERR_ARGUMENT, "%s: belief tensors must be 8-byte aligned", fn);
  for (const void* p : {(const void*)grad_q, (const void*)grad_k, (const void*)grad_v,
                        (const void*)grad_decay_logits, (const void*)grad_noise})
    if (p != nullptr && !aligned16(p))
      return fail(BSSM_ERR_ARGUMENT, "%s: the projection gradients must be 16-byte aligned", fn);
  bssm::MixArgs a{};
  a.q = q_proj; a.k = k_proj; a.v = v_proj; a.dl = decay_logits; a.nz = noise;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldd = ldd; a.ldn = ldn;
  a.m0 = mean0; a.c0 = cov0; a.bmr = bmean; a.bcr = bcov; a.gmf = gmf; a.gcf = gcf;
  a.gq = grad_q; a.gk = grad_k; a.gv = grad_v; a.gdl = grad_decay_logits; a.gnz = grad_noise;
  a.gm0 = gm0; a.gc0 = gc0;
  a.gate = gate; a.ldg = ldg; a.norm_w = norm_weight; a.norm_eps = norm_eps; a.yb = const_cast<void*>(read_bf16);
  a.gout = grad_out; a.ggate = grad_gate; a.gw_part = grad_norm_weight_partials;
  a.precise = precise != 0;
  a.grad_f32 = precise != 0;
  a.b = batch; a.t = t; a.h = heads; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = denominator_floor;
  if (n == 0) return ok();
  return launched(fn, bssm::launch_mixer_backward(a, static_cast<hipStream_t>(stream)));
}

namespace {
// The streams of config 4's Bayes block inside the fused projection
// [B, T, 30 H] (q, k, v core 16 H, decay logits 4 H, noise 2 H, gate 8 H per
// token) and the filtered core [B, T, 16 H]; the decay logits and noise are
// the projection's aux columns (the aux bias, if any, is added as they are
// read).
struct BlockStreams {
  const char *q, *k, *v, *dl, *nz, *gate;
  int64_t ldc;
  BlockStreams(const void* projected, const void* convolved, int64_t h) {
    const char* p = static_cast<const char*>(projected);
    const char* c = static_cast<const char*>(convolved);
    q = c;
    k = c + 2 * 4 * h;
    v = c + 2 * 8 * h;
    dl = p + 2 * 16 * h;
    nz = p + 2 * 20 * h;
    gate = p + 2 * 22 * h;
    ldc = 16 * h;
  }
};

int block_check(const char* fn, const void* projected, int64_t ld_projected, const float* conv_weight,
                const void* aux_bias, const void* convolved, int64_t b, int64_t t, int64_t h, int64_t chunk,
                float floor, const BlockStreams& s) {
  if (h <= 0 || b < 0) return fail(BSSM_ERR_ARGUMENT, "%s: needs heads > 0 and batch >= 0", fn);
  if (ld_projected < 30 * h)
    return fail(BSSM_ERR_ARGUMENT, "%s: the projection row stride must be >= 30 * heads = %lld (got %lld)", fn,
                (long long)(30 * h), (long long)ld_projected);
  if (b * t * h > 0 && (projected == nullptr || conv_weight == nullptr || convolved == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: projected, conv_weight and convolved are required (null given)", fn);
  if (aux_bias != nullptr && !aligned16(aux_bias))
    return fail(BSSM_ERR_ARGUMENT, "%s: aux_bias must be 16-byte aligned", fn);
  const int64_t ldp = ld_projected;
  if (int rc = mixer_check(fn, {s.q, s.k, s.v, s.dl, s.nz}, {s.ldc, s.ldc, s.ldc, ldp, ldp}, b, t, h, chunk, floor))
    return rc;
  if (int rc = conv_check(fn, 1, projected, ld_projected, conv_weight, {convolved}, b, t, 16 * h)) return rc;
  return BSSM_OK;
}
}  // namespace

int bssm_mixer_block_forward(const void* projected, int64_t ld_projected, const float* conv_weight,
                             const void* aux_bias, const float* norm_weight, float norm_eps, const float* mean0,
                             const float* cov0, void* convolved, void* out, void* read_bf16, float* mean_final,
                             float* cov_final, float* bmean, float* bcov, int64_t batch, int64_t t, int64_t heads,
                             int64_t chunk, float denominator_floor, void* stream) {
  const char* fn = "bssm_mixer_block_forward";
  const BlockStreams s(projected, convolved, heads);
  if (int rc = block_check(fn, projected, ld_projected, conv_weight, aux_bias, convolved, batch, t, heads, chunk,
                           denominator_floor, s))
    return rc;
  if (int rc = epilogue_check(fn, s.gate, ld_projected, norm_weight, norm_eps, {out, read_bf16}, batch, t, heads))
    return rc;
  const int64_t n = batch * heads;
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(mean_final);
  BSSM_REQUIRE(cov_final);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  for (const void* p : {(const void*)mean0, (const void*)cov0, (const void*)mean_final, (const void*)cov_final,
                        (const void*)bmean, (const void*)bcov})
    if (p != nullptr && !aligned8(p)) return fail(BSSM_ERR_ARGUMENT, "%s: belief tensors must be 8-byte aligned", fn);
  if (batch == 0) return ok();
  const hipStream_t st = static_cast<hipStream_t>(stream);
  bssm::ConvArgs c{};
  c.x = projected; c.ldx = ld_projected; c.w = conv_weight; c.y = convolved; c.b = batch; c.t = t; c.c = 16 * heads;
  c.bf16 = 1;
  if (hipError_t e = bssm::launch_conv4_forward(c, st); e != hipSuccess) return launched(fn, e);
  bssm::MixArgs a{};
  a.q = s.q; a.k = s.k; a.v = s.v; a.dl = s.dl; a.nz = s.nz;
  a.ldq = a.ldk = a.ldv = s.ldc; a.ldd = a.ldn = ld_projected; a.abias = aux_bias;
  a.m0 = mean0; a.c0 = cov0; a.mT = mean_final; a.cT = cov_final; a.bm = bmean; a.bc = bcov;
  a.gate = s.gate; a.ldg = ld_projected; a.norm_w = norm_weight; a.norm_eps = norm_eps; a.out = out;
  a.yb = read_bf16;
  a.b = batch; a.t = t; a.h = heads; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = denominator_floor;
  return launched(fn, bssm::launch_mixer_forward(a, st));
}

int bssm_mixer_block_backward(const void* projected, int64_t ld_projected, const float* conv_weight,
                              const void* aux_bias, const void* convolved, const float* norm_weight,
                              float norm_eps, const float* mean0, const float* cov0, const float* bmean,
                              const float* bcov, const void* read_bf16, const void* grad_out, const float* gmf,
                              const float* gcf, void* grad_convolved, void* grad_projected,
                              int64_t ld_grad_projected, float* grad_conv_weight_partials,
                              float* grad_norm_weight_partials, float* grad_aux_partials, void* grad_conv_weight,
                              void* grad_norm_weight, void* grad_aux_bias, int grad_bf16, float* gm0, float* gc0,
                              int64_t batch, int64_t t, int64_t heads, int64_t chunk, float denominator_floor,
                              void* stream) {
  const char* fn = "bssm_mixer_block_backward";
  const BlockStreams s(projected, convolved, heads);
  if (int rc = block_check(fn, projected, ld_projected, conv_weight, aux_bias, convolved, batch, t, heads, chunk,
                           denominator_floor, s))
    return rc;
  if (grad_aux_bias != nullptr && grad_aux_partials == nullptr)
    return fail(BSSM_ERR_ARGUMENT, "%s: grad_aux_bias needs the grad_aux_partials workspace", fn);
  if (int rc = epilogue_check(fn, s.gate, ld_projected, norm_weight, norm_eps,
                              {read_bf16, grad_out, grad_convolved, grad_norm_weight_partials,
                               grad_conv_weight_partials},
                              batch, t, heads))
    return rc;
  if (ld_grad_projected < 30 * heads || ld_grad_projected % 8 != 0 || !aligned16(grad_projected) ||
      (batch > 0 && grad_projected == nullptr))
    return fail(BSSM_ERR_ARGUMENT, "%s: grad_projected needs a 16-byte aligned base and a row stride >= 30 * heads, "
                "a multiple of 8 (got %lld)", fn, (long long)ld_grad_projected);
  if ((t + 16) * ld_grad_projected * 2 >= ((int64_t)1 << 31))
    return fail(BSSM_ERR_ARGUMENT, "%s: T * ld of grad_projected too large for 32-bit stream offsets", fn);
  const int64_t n = batch * heads;
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  for (const void* p : {(const void*)mean0, (const void*)cov0, (const void*)bmean, (const void*)bcov,
                        (const void*)gmf, (const void*)gcf, (const void*)gm0, (const void*)gc0})
    if (p != nullptr && !aligned8(p)) return fail(BSSM_ERR_ARGUMENT, "%s: belief tensors must be 8-byte aligned", fn);
  if (batch == 0) return ok();
  const hipStream_t st = static_cast<hipStream_t>(stream);
  char* gp = static_cast<char*>(grad_projected);
  char* gc = static_cast<char*>(grad_convolved);
  bssm::MixArgs a{};
  a.q = s.q; a.k = s.k; a.v = s.v; a.dl = s.dl; a.nz = s.nz;
  a.ldq = a.ldk = a.ldv = s.ldc; a.ldd = a.ldn = ld_projected; a.abias = aux_bias;
  a.m0 = mean0; a.c0 = cov0; a.bmr = bmean; a.bcr = bcov; a.gmf = gmf; a.gcf = gcf;
  a.gq = gc; a.gk = gc + 2 * 4 * heads; a.gv = gc + 2 * 8 * heads;
  a.gdl = gp + 2 * 16 * heads; a.gnz = gp + 2 * 20 * heads;
  a.ldgq = a.ldgk = a.ldgv = 16 * heads;
  a.ldgd = a.ldgn = a.ldgg = ld_grad_projected;
  a.gm0 = gm0; a.gc0 = gc0;
  a.gate = s.gate; a.ldg = ld_projected; a.norm_w = norm_weight; a.norm_eps = norm_eps;
  a.yb = const_cast<void*>(read_bf16); a.gout = grad_out; a.ggate = gp + 2 * 22 * heads;
  a.gw_part = grad_norm_weight_partials;
  a.b = batch; a.t = t; a.h = heads; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = denominator_floor;
  if (hipError_t e = bssm::launch_mixer_backward(a, st); e != hipSuccess) return launched(fn, e);
  bssm::ConvArgs c{};
  c.x = projected; c.ldx = ld_projected; c.w = conv_weight; c.gy = grad_convolved; c.gx = grad_projected;
  c.ldgx = ld_grad_projected; c.gw_part = grad_conv_weight_partials; c.b = batch; c.t = t; c.c = 16 * heads;
  c.bf16 = 1;
  if (hipError_t e = bssm::launch_conv4_backward(c, st); e != hipSuccess) return launched(fn, e);
  if (grad_aux_partials != nullptr) {
    if (hipError_t e = bssm::launch_column_sums_bf16(gp + 2 * 16 * heads, ld_grad_projected, batch, t, 6 * heads,
                                                     grad_aux_partials, st);
        e != hipSuccess)
      return launched(fn, e);
  }
  // The requested weight gradients: column sums of their partials.
  bssm::FoldArgs f{};
  const float* parts[3] = {grad_conv_weight_partials, grad_norm_weight_partials, grad_aux_partials};
  void* outs[3] = {grad_conv_weight, grad_norm_weight, grad_aux_bias};
  const int64_t rows[3] = {batch, batch * heads / 16, batch}, cols[3] = {16 * heads * 4, 8, 6 * heads};
  for (int i = 0; i < 3; ++i) {
    if (outs[i] == nullptr) continue;
    f.part[f.count] = parts[i];
    f.out[f.count] = outs[i];
    f.rows[f.count] = rows[i];
    f.cols[f.count] = cols[i];
    ++f.count;
  }
  f.bf16 = grad_bf16 != 0;
  return launched(fn, bssm::launch_fold(f, st));
}

int bssm_rotation_checkpoint(int key_dim) { return bssm::rotation_checkpoint(key_dim); }

int64_t bssm_small_batch_limit(int direction, int64_t limit) {
  if (direction < 0 || direction > 4) return -1;
  return limit >= 0 ? bssm::set_small_batch_limit(direction, limit) : bssm::small_batch_limit(direction);
}

namespace {
int rotation_common(const char* fn, int d, int m, int64_t n, int64_t t, int64_t chunk, float floor) {
  if (m != 8 || (d != 2 && d != 4 && d != 8))
    return fail(BSSM_ERR_UNSUPPORTED, "%s: rotation kernels support key_dim 2, 4, 8 with value_dim 8, got (%d, %d)",
                fn, d, m);
  if (n < 0 || t < 0) return fail(BSSM_ERR_ARGUMENT, "%s: negative size", fn);
  if (chunk <= 0) return fail(BSSM_ERR_ARGUMENT, "%s: chunk must be positive, got %lld", fn, (long long)chunk);
  if (!(floor > 0.f)) return fail(BSSM_ERR_ARGUMENT, "%s: denominator_floor must be positive", fn);
  if (n > (int64_t)0x7fffffff * 4 || t * 8 > ((int64_t)1 << 25))
    return fail(BSSM_ERR_ARGUMENT, "%s: n or t too large", fn);
  return BSSM_OK;
}
int rotation_vec(std::initializer_list<const void*> streams, int64_t t, int d) {
  for (const void* p : streams)
    if (p != nullptr && !aligned16(p)) return 0;
  return (t * (d / 2)) % 4 == 0 && t % 4 == 0;
}
}  // namespace

int bssm_forward_chunked_rotation(int key_dim, int value_dim, const float* keys, const float* values,
                                  const float* queries, const float* radii, const float* angles,
                                  const float* process, const float* observation, const float* mean0,
                                  const float* cov0, float* out, float* mean_final, float* cov_final, float* bmean,
                                  float* bcov, int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                  void* stream) {
  const char* fn = "bssm_forward_chunked_rotation";
  if (int rc = rotation_common(fn, key_dim, value_dim, n, t, chunk, denominator_floor)) return rc;
  BSSM_REQUIRE_T(keys);
  BSSM_REQUIRE_T(values);
  BSSM_REQUIRE_T(queries);
  BSSM_REQUIRE_T(radii);
  BSSM_REQUIRE_T(angles);
  BSSM_REQUIRE_T(process);
  BSSM_REQUIRE_T(observation);
  BSSM_REQUIRE_T(out);
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(mean_final);
  BSSM_REQUIRE(cov_final);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  bssm::RotArgs a{};
  a.k = keys; a.v = values; a.q = queries; a.rad = radii; a.ang = angles; a.p = process; a.r = observation;
  a.m0 = mean0; a.c0 = cov0; a.y = out; a.mT = mean_final; a.cT = cov_final; a.bm = bmean; a.bc = bcov;
  a.n = n; a.t = t; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = denominator_floor;
  a.vec = rotation_vec({keys, values, queries, radii, angles, process, observation, out}, t, key_dim);
  if (n == 0) return ok();
  return launched(fn, bssm::launch_rotation_forward(key_dim, a, static_cast<hipStream_t>(stream)));
}

int bssm_backward_chunked_rotation(int key_dim, int value_dim, const float* keys, const float* values,
                                   const float* queries, const float* radii, const float* angles,
                                   const float* process, const float* observation, const float* mean0,
                                   const float* cov0, const float* bmean, const float* bcov, const float* gy,
                                   const float* gmf, const float* gcf, float* gk, float* gv, float* gq,
                                   float* g_radii, float* g_angles, float* g_process, float* g_observation,
                                   float* gm0, float* gc0, int64_t n, int64_t t, int64_t chunk,
                                   float denominator_floor, void* stream) {
  const char* fn = "bssm_backward_chunked_rotation";
  if (int rc = rotation_common(fn, key_dim, value_dim, n, t, chunk, denominator_floor)) return rc;
  BSSM_REQUIRE_T(keys);
  BSSM_REQUIRE_T(values);
  BSSM_REQUIRE_T(queries);
  BSSM_REQUIRE_T(radii);
  BSSM_REQUIRE_T(angles);
  BSSM_REQUIRE_T(process);
  BSSM_REQUIRE_T(observation);
  BSSM_REQUIRE_T(gy);
  BSSM_REQUIRE(bmean);
  BSSM_REQUIRE(bcov);
  BSSM_REQUIRE_T(gk);
  BSSM_REQUIRE_T(gv);
  BSSM_REQUIRE_T(gq);
  BSSM_REQUIRE_T(g_radii);
  BSSM_REQUIRE_T(g_angles);
  BSSM_REQUIRE_T(g_process);
  BSSM_REQUIRE_T(g_observation);
  bssm::RotArgs a{};
  a.k = keys; a.v = values; a.q = queries; a.rad = radii; a.ang = angles; a.p = process; a.r = observation;
  a.m0 = mean0; a.c0 = cov0; a.bm = const_cast<float*>(bmean); a.bc = const_cast<float*>(bcov);
  a.gy = gy; a.gmf = gmf; a.gcf = gcf;
  a.gk = gk; a.gv = gv; a.gq = gq; a.grad = g_radii; a.gang = g_angles; a.gp = g_process; a.gr = g_observation;
  a.gm0 = gm0; a.gc0 = gc0;
  a.n = n; a.t = t; a.chunk = chunk; a.nb = (t + chunk - 1) / chunk; a.floor = denominator_floor;
  a.vec = rotation_vec({keys, values, queries, radii, angles, process, observation, gy, gk, gv, gq, g_radii,
                        g_angles, g_process, g_observation}, t, key_dim);
  if (n == 0) return ok();
  return launched(fn, bssm::launch_rotation_backward(key_dim, a, static_cast<hipStream_t>(stream)));
}

int bssm_causal_conv4_forward(int bf16, const void* x, int64_t ldx, const float* weight, void* y, int64_t batch,
                              int64_t t, int64_t channels, void* stream) {
  const char* fn = "bssm_causal_conv4_forward";
  if (int rc = conv_check(fn, bf16, x, ldx, weight, {y}, batch, t, channels)) return rc;
  bssm::ConvArgs a{};
  a.x = x; a.ldx = ldx; a.w = weight; a.y = y; a.b = batch; a.t = t; a.c = channels; a.bf16 = bf16 != 0;
  if (batch * t * channels == 0) return ok();
  return launched(fn, bssm::launch_conv4_forward(a, static_cast<hipStream_t>(stream)));
}

int bssm_causal_conv4_backward(int bf16, const void* x, int64_t ldx, const float* weight, const void* grad_y,
                               void* grad_x, float* grad_weight_partials, int64_t batch, int64_t t,
                               int64_t channels, void* stream) {
  const char* fn = "bssm_causal_conv4_backward";
  if (int rc = conv_check(fn, bf16, x, ldx, weight, {grad_y, grad_x, grad_weight_partials}, batch, t, channels))
    return rc;
  // With T = 0 the kernel still reads the weight and writes zero partials.
  if (batch * channels > 0 && (weight == nullptr || grad_weight_partials == nullptr || !aligned16(weight) ||
                               !aligned16(grad_weight_partials)))
    return fail(BSSM_ERR_ARGUMENT, "%s: weight and grad_weight_partials must be non-null and 16-byte aligned", fn);
  bssm::ConvArgs a{};
  a.x = x; a.ldx = ldx; a.w = weight; a.gy = grad_y; a.gx = grad_x; a.gw_part = grad_weight_partials;
  a.b = batch; a.t = t; a.c = channels; a.bf16 = bf16 != 0;
  if (batch * channels == 0) return ok();
  return launched(fn, bssm::launch_conv4_backward(a, static_cast<hipStream_t>(stream)));
}

int bssm_causal_conv4_backward_noalloc(int bf16, const void* x, int64_t ldx, const float* weight,
                                       const void* grad_y, void* grad_x, float* grad_weight, int64_t batch,
                                       int64_t t, int64_t channels, void* stream) {
  const char* fn = "bssm_causal_conv4_backward_noalloc";
  if (int rc = conv_check(fn, bf16, x, ldx, weight, {grad_y, grad_x}, batch, t, channels)) return rc;
  if (batch * channels * 4 > bssm::kConv4ScratchFloats)
    return fail(BSSM_ERR_ARGUMENT, "%s: batch * channels = %lld exceeds the library scratch (at most %lld)", fn,
                (long long)(batch * channels), (long long)(bssm::kConv4ScratchFloats / 4));
  if (channels == 0) return ok();
  // grad_weight is written (zeros without batch entries or tokens); the
  // kernels read the weight whenever there are batch entries.
  if (grad_weight == nullptr || !aligned16(grad_weight) || (batch > 0 && (weight == nullptr || !aligned16(weight))))
    return fail(BSSM_ERR_ARGUMENT, "%s: weight and grad_weight must be non-null and 16-byte aligned", fn);
  bssm::ConvArgs a{};
  a.x = x; a.ldx = ldx; a.w = weight; a.gy = grad_y; a.gx = grad_x; a.gw_part = nullptr;
  a.b = batch; a.t = t; a.c = channels; a.bf16 = bf16 != 0;
  return launched(fn, bssm::launch_conv4_backward_noalloc(a, grad_weight, static_cast<hipStream_t>(stream)));
}

int bssm_associative_static_scan(const float* keys, const float* values, const float* queries,
                                 const float* observation, const float* mean0, const float* cov0, float* out,
                                 float* mean_final, float* cov_final, int64_t b, int64_t t, int key_dim,
                                 int value_dim, void* stream) {
  const char* fn = "bssm_associative_static_scan";
  if (key_dim <= 0 || key_dim > 32 || value_dim <= 0 || value_dim > 64)
    return fail(BSSM_ERR_UNSUPPORTED, "%s: needs 0 < key_dim <= 32 and 0 < value_dim <= 64, got (%d, %d)", fn,
                key_dim, value_dim);
  if (b < 0 || t < 0) return fail(BSSM_ERR_ARGUMENT, "%s: negative size", fn);
  if (b > 65535 || t > 0x7fffffff) return fail(BSSM_ERR_ARGUMENT, "%s: b or t too large", fn);
  const int64_t n = b;
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(mean_final);
  BSSM_REQUIRE(cov_final);
  BSSM_REQUIRE_T(keys);
  BSSM_REQUIRE_T(values);
  BSSM_REQUIRE_T(queries);
  BSSM_REQUIRE_T(observation);
  BSSM_REQUIRE_T(out);
  return launched(fn, bssm::launch_associative_scan(keys, values, queries, observation, mean0, cov0, out, mean_final,
                                                    cov_final, b, t, key_dim, value_dim,
                                                    static_cast<hipStream_t>(stream)));
}

int bssm_associative_static_scan_backward(const float* keys, const float* values, const float* queries,
                                          const float* observation, const float* mean0, const float* cov0,
                                          const float* grad_out, const float* grad_mean_final,
                                          const float* grad_cov_final, float* workspace, float* grad_keys,
                                          float* grad_values, float* grad_queries, float* grad_observation,
                                          float* grad_mean0, float* grad_cov0, int64_t b, int64_t t, int key_dim,
                                          int value_dim, void* stream) {
  const char* fn = "bssm_associative_static_scan_backward";
  if (key_dim <= 0 || key_dim > bssm::kMaxBackwardD || value_dim <= 0 || value_dim > 64)
    return fail(BSSM_ERR_UNSUPPORTED, "%s: needs 0 < key_dim <= %d and 0 < value_dim <= 64, got (%d, %d)", fn,
                bssm::kMaxBackwardD, key_dim, value_dim);
  if (b < 0 || t <= 0) return fail(BSSM_ERR_ARGUMENT, "%s: needs b >= 0 and t >= 1", fn);
  if (b > 65535 || t > 0x7fffffff) return fail(BSSM_ERR_ARGUMENT, "%s: b or t too large", fn);
  const int64_t n = b;
  BSSM_REQUIRE(keys);
  BSSM_REQUIRE(values);
  BSSM_REQUIRE(queries);
  BSSM_REQUIRE(observation);
  BSSM_REQUIRE(mean0);
  BSSM_REQUIRE(cov0);
  BSSM_REQUIRE(grad_out);
  BSSM_REQUIRE(workspace);
  BSSM_REQUIRE(grad_keys);
  BSSM_REQUIRE(grad_values);
  BSSM_REQUIRE(grad_queries);
  BSSM_REQUIRE(grad_observation);
  BSSM_REQUIRE(grad_mean0);
  BSSM_REQUIRE(grad_cov0);
  return launched(fn, bssm::launch_associative_scan_backward(
                          keys, values, queries, observation, mean0, cov0, grad_out, grad_mean_final, grad_cov_final,
                          workspace, grad_keys, grad_values, grad_queries, grad_observation, grad_mean0, grad_cov0, b,
                          t, key_dim, value_dim, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
