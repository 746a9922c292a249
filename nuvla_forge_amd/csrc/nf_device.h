// Device-side helpers shared by the gfx950 kernels: element I/O in 8-wide
// chunks (one 16-byte load for bf16/f16, two for f32), dtype-tagged scalar
// loads for small conditioning tensors, and wavefront reductions built on DPP
// row operations.  All arithmetic is fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nuvla_forge_hip.h"

namespace nf {

using bf16 = __bf16;
using f16 = _Float16;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// scalar conversions (hardware RNE conversions on gfx950)
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return static_cast<float>(v);
}
template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return static_cast<T>(v);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// ---------------------------------------------------------------------------
// Streamed loads: activation data that a row / elementwise kernel reads once.
// NTL adds the non-temporal hint.  The hint pays only when a launch streams
// more input than the 256 MB Infinity Cache holds; below that it costs.  A/B
// on one MI355X (bf16, warm back-to-back launches, outputs bit-identical),
// plain -> hinted, by the launch's streamed input bytes:
//   adaLN fwd   34 / 134 / 268 / 402 / 537 MB: 10.5 -> 13.0, 45.0 -> 49.7,
//               89.6 -> 97.7, 148 -> 142, 190 -> 181 us;
//   adaLN bwd   67 / 268 / 537 / 1074 MB: 18.7 -> 19.7, 76.6 -> 76.7,
//               161 -> 150, 304 -> 298 us;
//   SwiGLU fwd  134 / 268 / 370 / 738 / 1476 MB: 29.2 -> 30.7, 56.3 -> 60.1,
//               90.7 -> 82.7, 183 -> 167, 353 -> 327 us;
//   SwiGLU bwd  201 / 402 / 555 / 1107 / 2214 MB: 48.1 -> 53.7,
//               112.6 -> 105.2, 152.4 -> 142.0, 313 -> 292, 599 -> 562 us.
// So a launch takes the hint when its streamed inputs exceed kNtLoadMinBytes
// (between the largest size where it lost and the smallest where it won).
// ---------------------------------------------------------------------------
constexpr int64_t kNtLoadMinBytes = (int64_t)320 << 20;
inline bool nt_loads_for(int64_t input_bytes) { return input_bytes > kNtLoadMinBytes; }

template <bool NTL>
__device__ __forceinline__ u32x4 stream_load16(const void *p) {
  if constexpr (NTL)
    return __builtin_nontemporal_load(static_cast<const u32x4 *>(p));
  else
    return *static_cast<const u32x4 *>(p);
}

// A 16- or 32-byte vector type V loaded as whole 16-byte streamed loads.
template <typename V, bool NTL>
__device__ __forceinline__ V stream_load_vec(const void *p) {
  static_assert(sizeof(V) == 16 || sizeof(V) == 32, "16- or 32-byte vectors");
  if constexpr (sizeof(V) == 16) {
    return __builtin_bit_cast(V, stream_load16<NTL>(p));
  } else {
    const u32x4 a = stream_load16<NTL>(p);
    const u32x4 b = stream_load16<NTL>(static_cast<const char *>(p) + 16);
    return __builtin_bit_cast(V, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
  }
}

// ---------------------------------------------------------------------------
// 8-element chunk I/O.  `p` must be 16-byte aligned for the vector forms.
// ---------------------------------------------------------------------------
template <typename T>
struct Chunk8;

template <>
struct Chunk8<float> {
  __device__ __forceinline__ static void load(const float *p, float (&v)[8]) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(p);
    const u32x4 b = *reinterpret_cast<const u32x4 *>(p + 4);
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
    v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y);
    v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
  }
  __device__ __forceinline__ static void store(float *p, const float (&v)[8]) {
    u32x4 a, b;
    a.x = __float_as_uint(v[0]); a.y = __float_as_uint(v[1]);
    a.z = __float_as_uint(v[2]); a.w = __float_as_uint(v[3]);
    b.x = __float_as_uint(v[4]); b.y = __float_as_uint(v[5]);
    b.z = __float_as_uint(v[6]); b.w = __float_as_uint(v[7]);
    *reinterpret_cast<u32x4 *>(p) = a;
    *reinterpret_cast<u32x4 *>(p + 4) = b;
  }
};

template <typename T16>
struct Chunk8Half {
  __device__ __forceinline__ static void load(const T16 *p, float (&v)[8]) {
    typedef T16 t16x8 __attribute__((ext_vector_type(8)));
    const t16x8 a = *reinterpret_cast<const t16x8 *>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(a[i]);
  }
  __device__ __forceinline__ static void store(T16 *p, const float (&v)[8]) {
    typedef T16 t16x8 __attribute__((ext_vector_type(8)));
    t16x8 a;
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = static_cast<T16>(v[i]);
    *reinterpret_cast<t16x8 *>(p) = a;
  }
};
template <>
struct Chunk8<bf16> : Chunk8Half<bf16> {};
template <>
struct Chunk8<f16> : Chunk8Half<f16> {};

// Masked element-wise chunk I/O for rows whose length is not a multiple of 8
// or whose pointers are not 16-byte aligned.  Elements at or past `valid`
// read as zero and are not written.
template <typename T>
__device__ __forceinline__ void load8_masked(const T *p, int valid,
                                             float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (i < valid) ? to_f32(p[i]) : 0.f;
}
template <typename T>
__device__ __forceinline__ void store8_masked(T *p, int valid,
                                              const float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < valid) p[i] = from_f32<T>(v[i]);
}

template <typename T, bool VEC>
__device__ __forceinline__ void load8(const T *p, int valid, float (&v)[8]) {
  if (VEC && valid >= 8)
    Chunk8<T>::load(p, v);
  else
    load8_masked<T>(p, valid, v);
}
template <typename T, bool VEC>
__device__ __forceinline__ void store8(T *p, int valid, const float (&v)[8]) {
  if (VEC && valid >= 8)
    Chunk8<T>::store(p, v);
  else
    store8_masked<T>(p, valid, v);
}

// As store8, with the non-temporal hint on the 16-byte vector stores when NT
// (streaming outputs that are not re-read by this kernel).
template <typename T, bool VEC, bool NT>
__device__ __forceinline__ void store8_hint(T *p, int valid, const float (&v)[8]) {
  if constexpr (NT) {
    if (VEC && valid >= 8) {
      if constexpr (sizeof(T) == 4) {
        u32x4 a, b;
        a.x = __float_as_uint(v[0]); a.y = __float_as_uint(v[1]);
        a.z = __float_as_uint(v[2]); a.w = __float_as_uint(v[3]);
        b.x = __float_as_uint(v[4]); b.y = __float_as_uint(v[5]);
        b.z = __float_as_uint(v[6]); b.w = __float_as_uint(v[7]);
        __builtin_nontemporal_store(a, reinterpret_cast<u32x4 *>(p));
        __builtin_nontemporal_store(b, reinterpret_cast<u32x4 *>(p + 4));
      } else {
        typedef T t8 __attribute__((ext_vector_type(8)));
        t8 a;
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = static_cast<T>(v[i]);
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, a), reinterpret_cast<u32x4 *>(p));
      }
      return;
    }
  }
  store8<T, VEC>(p, valid, v);
}

// An 8-element chunk kept in its storage type (4 VGPRs for bf16/f16, 8 for
// f32) and widened to fp32 element by element on use.  Holding a row's
// incoming chunks this way halves the register cost of 16-bit inputs.
template <typename T>
struct Raw8 {
  typedef T vtype __attribute__((ext_vector_type(8)));
  vtype v;
  __device__ __forceinline__ float operator[](int i) const {
    return static_cast<float>(v[i]);
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<T>(0.f);
  }
  template <bool VEC, bool NTL = false>
  __device__ __forceinline__ void load(const T *p, int valid) {
    if (VEC && valid >= 8) {
      v = stream_load_vec<vtype, NTL>(p);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = i < valid ? p[i] : static_cast<T>(0.f);
    }
  }
};

// load8 for streamed activation data: the vector form goes through
// stream_load16<NTL>.
template <typename T, bool VEC, bool NTL>
__device__ __forceinline__ void load8_stream(const T *p, int valid, float (&v)[8]) {
  if (VEC && valid >= 8) {
    Raw8<T> r;
    r.template load<true, NTL>(p, 8);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = r[i];
  } else {
    load8_masked<T>(p, valid, v);
  }
}

// Runtime-typed chunk load for the small [B, N] / [N] conditioning tensors
// (their element type may differ from the activations').  `dt` is uniform
// across the wavefront, so the switch does not diverge.
template <bool VEC>
__device__ __forceinline__ void load8_dyn(const void *p, int dt, int64_t off,
                                          int valid, float (&v)[8]) {
  if (dt == NF_DTYPE_F32)
    load8<float, VEC>(static_cast<const float *>(p) + off, valid, v);
  else if (dt == NF_DTYPE_BF16)
    load8<bf16, VEC>(static_cast<const bf16 *>(p) + off, valid, v);
  else
    load8<f16, VEC>(static_cast<const f16 *>(p) + off, valid, v);
}

__device__ __forceinline__ void store_dyn(void *p, int dt, int64_t off,
                                          float v) {
  if (dt == NF_DTYPE_F32)
    static_cast<float *>(p)[off] = v;
  else if (dt == NF_DTYPE_BF16)
    static_cast<bf16 *>(p)[off] = static_cast<bf16>(v);
  else
    static_cast<f16 *>(p)[off] = static_cast<f16>(v);
}

// ---------------------------------------------------------------------------
// Wavefront reductions.  Steps inside a 16-lane DPP row use quad_perm and the
// row mirrors (each pairs every lane with a partner in the other half of its
// group, so after four steps all 16 lanes hold the row total); the two
// cross-row steps use ds_swizzle (xor 16 inside 32 lanes) and a readlane pair.
// Every lane returns the same value, and the order of additions is fixed, so
// the result is bit-reproducible.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]: partner = lane ^ 1
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]: partner = lane ^ 2
  v += dpp<0x141>(v);  // row_half_mirror: lane i <-> 7 - i within 8
  v += dpp<0x140>(v);  // row_mirror:      lane i <-> 15 - i within 16
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return lo + hi;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return fmaxf(lo, hi);
}

// Reductions over the 32 lanes that share (lane / 32): the column axis of a
// 32x32 MFMA accumulator.  Every lane of each half gets its half's result.
__device__ __forceinline__ float half_wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  return v;
}
__device__ __forceinline__ float half_wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));
  return v;
}

// sigmoid(a) = 1 / (1 + e^-a) with e^-a = 2^(-a * log2(e)) on the hardware
// exp2 and the hardware reciprocal.  Saturates cleanly: a -> -inf gives
// 2^+inf = inf and 1/inf = 0; a -> +inf gives 1/(1+0) = 1.
__device__ __forceinline__ float sigmoid(float a) {
  constexpr float kLog2e = 1.4426950408889634f;  // log2(e)
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-a * kLog2e));
}

__device__ __forceinline__ float exp_f32(float x) {
  constexpr float kLog2e = 1.4426950408889634f;
  return __builtin_amdgcn_exp2f(x * kLog2e);
}

}  // namespace nf

// ---------------------------------------------------------------------------
// host-side error plumbing (defined in nf_common.hip)
// ---------------------------------------------------------------------------
namespace nf {
int set_error(int code, const char *fmt, ...);
int check_launch(const char *what);
inline bool is_dtype(int dt) {
  return dt == NF_DTYPE_F32 || dt == NF_DTYPE_BF16 || dt == NF_DTYPE_F16;
}
inline bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}
}  // namespace nf
