// Shared device helpers for the gfx950 body kernels: element I/O in 8-element chunks and
// wavefront reductions on DPP.
//
// Data layout convention of every kernel here: a row (or a head half) is cut into chunks of
// 8 consecutive elements. A lane always owns whole chunks, so a 16-bit chunk is one 16-byte
// buffer_load_dwordx4 and an fp32 chunk is two. The chunk -> lane mapping is the same for
// every element type, which is what lets fp32 residuals mix with 16-bit deltas and outputs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace esep {

constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------
// Scalar conversions. bf16 -> fp32 is exact (a shift); fp32 -> bf16 and fp32 -> fp16 round to
// nearest even (the compiler lowers __bf16 / _Float16 truncation to the hardware converts).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <typename T> struct Elt;
template <> struct Elt<float> {
  static constexpr int kBytes = 4;
  __device__ static float to_f(float v) { return v; }
  __device__ static float from_f(float v) { return v; }
  __device__ static float round(float v) { return v; }
};
template <> struct Elt<_Float16> {
  static constexpr int kBytes = 2;
  __device__ static float to_f(_Float16 v) { return (float)v; }
  __device__ static _Float16 from_f(float v) { return (_Float16)v; }
  __device__ static float round(float v) { return (float)(_Float16)v; }
};
template <> struct Elt<__bf16> {
  static constexpr int kBytes = 2;
  __device__ static float to_f(__bf16 v) { return (float)v; }
  __device__ static __bf16 from_f(float v) { return (__bf16)v; }
  __device__ static float round(float v) { return (float)(__bf16)v; }
};

template <typename T> constexpr bool kLowp = Elt<T>::kBytes == 2;

// ---------------------------------------------------------------------------------------
// Row I/O through buffer resources. A row (or any wave-uniform span) gets a 128-bit buffer
// descriptor in SGPRs whose record count is the span's size in bytes; every access is an
// `offen` buffer instruction with a 32-bit lane offset. The hardware range check returns 0
// for a read past the end and drops a write past the end, so ragged tails and rows past the
// last one need no branches (a row beyond the tensor gets a 0-byte descriptor).
// ---------------------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Descriptor word 3 for gfx9-family raw buffers (32-bit data format, no swizzle).
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}

// Cache policy of a buffer access (the instruction's cache-policy bits on gfx950):
// kCached for data that is re-read (norm weights, slot tables), kStream (nt: non-temporal)
// for tensors that are read or written exactly once per kernel.
constexpr int kCached = 0;
constexpr int kStream = 2;

template <int POL = kCached>
__device__ __forceinline__ u32x4 buf_ld16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL);
}
template <int POL = kCached>
__device__ __forceinline__ void buf_st16(rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, POL);
}

// A row (or other wave-uniform span): its buffer descriptor, base pointer and size in bytes.
struct Span {
  rsrc_t r;
  const char* p;
  uint32_t bytes;
};

__device__ __forceinline__ Span make_span(const void* base, uint32_t bytes) {
  return Span{make_rsrc(base, bytes), static_cast<const char*>(base), bytes};
}

// Raw (still packed) contents of one 8-element chunk: 16 bytes for 16-bit types, 32 for fp32.
// Loading raw and unpacking at the point of use keeps a prefetched 16-bit chunk in 4 VGPRs
// instead of 8.
template <typename T> struct Raw {
  u32x4 a;
};
template <> struct Raw<float> {
  u32x4 a, b;
};

// 8 consecutive elements starting at byte offset `off` of the span. VEC: two (fp32) or one
// (16-bit) 16-byte buffer accesses; the span base and `off` are 16-byte aligned and the chunk
// is whole or wholly outside. !VEC (ragged or unaligned rows, the rare path): one
// bounds-checked pointer access per element.
template <typename T> struct Buf {
  typedef T v8 __attribute__((ext_vector_type(8)));

  template <int POL>
  __device__ static Raw<T> load_raw(const Span& s, uint32_t off) {
    Raw<T> r;
    r.a = buf_ld16<POL>(s.r, off);
    if constexpr (sizeof(T) == 4) r.b = buf_ld16<POL>(s.r, off + 16);
    return r;
  }

  __device__ static void unpack(const Raw<T>& r, float (&v)[8]) {
    if constexpr (sizeof(T) == 4) {
      v[0] = __uint_as_float(r.a.x); v[1] = __uint_as_float(r.a.y);
      v[2] = __uint_as_float(r.a.z); v[3] = __uint_as_float(r.a.w);
      v[4] = __uint_as_float(r.b.x); v[5] = __uint_as_float(r.b.y);
      v[6] = __uint_as_float(r.b.z); v[7] = __uint_as_float(r.b.w);
    } else if constexpr (std::is_same_v<T, __bf16>) {
      v[0] = bf16_lo(r.a.x); v[1] = bf16_hi(r.a.x);
      v[2] = bf16_lo(r.a.y); v[3] = bf16_hi(r.a.y);
      v[4] = bf16_lo(r.a.z); v[5] = bf16_hi(r.a.z);
      v[6] = bf16_lo(r.a.w); v[7] = bf16_hi(r.a.w);
    } else {
      const v8 h = __builtin_bit_cast(v8, r.a);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (float)h[e];
    }
  }

  template <bool VEC, int POL = kCached>
  __device__ static void load(const Span& s, uint32_t off, float (&v)[8]) {
    if constexpr (VEC) {
      unpack(load_raw<POL>(s, off), v);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t o = off + e * (uint32_t)sizeof(T);
        v[e] = o < s.bytes ? Elt<T>::to_f(*reinterpret_cast<const T*>(s.p + o)) : 0.f;
      }
    }
  }

  template <bool VEC, int POL = kCached>
  __device__ static void store(const Span& s, uint32_t off, const float (&v)[8]) {
    if constexpr (VEC) {
      if constexpr (sizeof(T) == 4) {
        buf_st16<POL>(s.r, off, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]),
                                      __float_as_uint(v[2]), __float_as_uint(v[3])});
        buf_st16<POL>(s.r, off + 16, u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]),
                                           __float_as_uint(v[6]), __float_as_uint(v[7])});
      } else {
        v8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = Elt<T>::from_f(v[e]);
        buf_st16<POL>(s.r, off, __builtin_bit_cast(u32x4, h));
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t o = off + e * (uint32_t)sizeof(T);
        if (o < s.bytes) *reinterpret_cast<T*>(const_cast<char*>(s.p) + o) = Elt<T>::from_f(v[e]);
      }
    }
  }
};

// int32 chunk (slot table of the exact channels); elements past the span read -1.
template <bool VEC>
__device__ __forceinline__ void buf_load8_i32(const Span& s, uint32_t off, int (&v)[8]) {
  if constexpr (VEC) {
    const u32x4 a = buf_ld16(s.r, off), b = buf_ld16(s.r, off + 16);
    const bool in = off < s.bytes;
    v[0] = in ? (int)a.x : -1; v[1] = in ? (int)a.y : -1;
    v[2] = in ? (int)a.z : -1; v[3] = in ? (int)a.w : -1;
    v[4] = in ? (int)b.x : -1; v[5] = in ? (int)b.y : -1;
    v[6] = in ? (int)b.z : -1; v[7] = in ? (int)b.w : -1;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t o = off + 4u * e;
      v[e] = o < s.bytes ? *reinterpret_cast<const int*>(s.p + o) : -1;
    }
  }
}

// Plain-pointer 8-element chunk access (16-byte aligned), used where the span is not a row.
template <typename T> struct Chunk;

template <> struct Chunk<float> {
  __device__ static void load(const float* p, float (&v)[8]) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  __device__ static void store(float* p, const float (&v)[8]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
};

template <> struct Chunk<_Float16> {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  __device__ static void load(const _Float16* p, float (&v)[8]) {
    const h8 h = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)h[e];
  }
  __device__ static void store(_Float16* p, const float (&v)[8]) {
    h8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (_Float16)v[e];
    *reinterpret_cast<h8*>(p) = h;
  }
};

template <> struct Chunk<__bf16> {
  typedef __bf16 b8 __attribute__((ext_vector_type(8)));
  __device__ static void load(const __bf16* p, float (&v)[8]) {
    const u32x4 u = *reinterpret_cast<const u32x4*>(p);
    v[0] = bf16_lo(u.x); v[1] = bf16_hi(u.x);
    v[2] = bf16_lo(u.y); v[3] = bf16_hi(u.y);
    v[4] = bf16_lo(u.z); v[5] = bf16_hi(u.z);
    v[6] = bf16_lo(u.w); v[7] = bf16_hi(u.w);
  }
  __device__ static void store(__bf16* p, const float (&v)[8]) {
    b8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (__bf16)v[e];
    *reinterpret_cast<b8*>(p) = h;
  }
};

// Index of this thread's wavefront within the block, as a wave-uniform (SGPR) value.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------------------
// Wavefront sum on DPP. Every lane ends with the same bits: each step adds a lane and its
// partner (commutative), and the last step combines the four 16-lane rows in a fixed order
// through readlane. The order depends on nothing but the lane layout, so it is reproducible.
// ---------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  v += dpp_f<0x141>(v);  // row_half_mirror: the other quad of each 8
  v += dpp_f<0x140>(v);  // row_mirror: the other half of each 16-lane row
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Wave-scope ordering for a wave that writes LDS and then reads what other lanes wrote.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace esep
