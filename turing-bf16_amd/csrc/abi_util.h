// Host-side helpers shared by the C-ABI entry points: thread-local error text,
// precondition checks and launch checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tbf16_hip.h"

namespace tbf16 {

void set_error(const char* fmt, ...);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Attention dropout parameters: thr16 = round(p * 65536), at least 1 for p > 0 and
// 0 for no dropout; scale = 1 / (1 - p); the seed's two halves are the mixing words.
inline void set_dropout(float p, uint64_t seed, uint32_t& lo, uint32_t& hi, uint32_t& thr16, float& scale) {
  double t = (double)p * 65536.0 + 0.5;
  if (t > 65535.0) t = 65535.0;
  thr16 = p > 0.f ? (uint32_t)t : 0u;
  if (p > 0.f && thr16 == 0u) thr16 = 1u;
  scale = thr16 ? 1.f / (1.f - p) : 1.f;
  lo = (uint32_t)seed;
  hi = (uint32_t)(seed >> 32);
}

// One (B, H, S, D) bf16 tensor of a multi-tensor head-amax launch: BH = B * H heads,
// strides sb / sh / ss, nch chunks of rows rows each, maxima into partial[bh * nch + c].
struct AmaxSeg {
  const uint16_t* x;
  int64_t BH, H, S, sb, sh, ss, rows, nch;
  float* partial;
};
struct AmaxSegs {
  AmaxSeg seg[3];
  int n;
};
int launch_head_amax3(const AmaxSegs& segs, int64_t D, hipStream_t st);

}  // namespace tbf16

#define TB_CHECK(cond, ...)           \
  do {                                \
    if (!(cond)) {                    \
      ::tbf16::set_error(__VA_ARGS__); \
      return TBF16_EINVAL;            \
    }                                 \
  } while (0)

#define TB_LAUNCH_CHECK(name)                                                                 \
  do {                                                                                        \
    hipError_t e_ = hipGetLastError();                                                        \
    if (e_ != hipSuccess) {                                                                   \
      ::tbf16::set_error("%s: kernel launch failed: %s", name, hipGetErrorString(e_));       \
      return TBF16_ELAUNCH;                                                                   \
    }                                                                                         \
  } while (0)
