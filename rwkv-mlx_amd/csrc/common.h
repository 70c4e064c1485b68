// Shared device-side helpers for the gfx950 kernels of librwkvmoe.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef __bf16 bf16;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

#define RWKV_DEV __device__ __forceinline__

// Kernel arguments come through the scalar cache, and the compiler loads each
// one where it is first used: a kernel whose arguments span several 64-byte
// lines can wait for one cold line after another (about 0.7 us each).  Naming
// one argument from every line at entry — an empty asm that needs them in
// SGPRs — has all the lines fetched together, behind a single wait.
#define RWKV_KERNARG_LINES(...) asm volatile("" ::__VA_ARGS__)

// Round a float to the element type T and back: the rounding point the
// reference applies after every op on T-typed arrays.
template <typename T> RWKV_DEV float rnd(float v) { return (float)(T)v; }
template <> RWKV_DEV float rnd<float>(float v) { return v; }

template <typename T> RWKV_DEV float to_f(T v) { return (float)v; }
template <typename T> RWKV_DEV T from_f(float v) { return (T)v; }

// 16-byte chunk <-> elements.
template <typename T> struct Chunk {
  static constexpr int N = 16 / sizeof(T);
  union {
    u32x4 raw;
    T e[N];
  };
};

RWKV_DEV u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

// The token-shift mix of one 16-byte chunk, xk = x + round(round(prev - x)
// · x_k), each op rounded to T (model.py:260-261).  fp16 runs it as packed
// fp16 arithmetic: one IEEE rounding per op, the same values as each op
// computed in fp32 and rounded to fp16 (the difference of two fp16 values
// and the product of two are exact in fp32, and an fp32 sum of two fp16
// values never rounds onto an fp16 midpoint it was not already on).
template <typename T>
RWKV_DEV u32x4 shift_mix_chunk(u32x4 x, u32x4 prev, u32x4 mu) {
  Chunk<T> xc, pc, mc, o;
  xc.raw = x;
  pc.raw = prev;
  mc.raw = mu;
#pragma unroll
  for (int j = 0; j < Chunk<T>::N; ++j) {
    const float xf = to_f(xc.e[j]);
    const float xx = rnd<T>(to_f(pc.e[j]) - xf);
    o.e[j] = from_f<T>(xf + rnd<T>(xx * to_f(mc.e[j])));
  }
  return o.raw;
}
template <>
RWKV_DEV u32x4 shift_mix_chunk<f16>(u32x4 x, u32x4 prev, u32x4 mu) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 xv = __builtin_bit_cast(h8, x), pv = __builtin_bit_cast(h8, prev), mv = __builtin_bit_cast(h8, mu);
  const h8 xx = pv - xv;
  const h8 t = xx * mv;
  return __builtin_bit_cast(u32x4, xv + t);
}

// Fragment order of a (rows x C) 16-bit matrix (rows a multiple of 16, C of
// 32) for v_mfma_f32_16x16x32 operands: the 8 elements a lane l feeds for
// 16-row block b and k-step j — (b·16 + l % 16, j·32 + (l / 16)·8 + 0..7) —
// sit at position ((b·C/32 + j)·64 + l)·8, so a wave's fragment is 1 KB
// contiguous.  frag_pos gives the position of element (row, c).
RWKV_DEV size_t frag_pos(int row, int c, int C) {
  return ((((size_t)(row >> 4) * (C >> 5) + (c >> 5)) * 64 + (row & 15) + 16 * ((c & 31) >> 3)) << 3) + (c & 7);
}

// Fragment order with two operands per K-step (fp32 adapters carried as
// fp16 pairs, pass 0 = hi, pass 1 = lo'): position of element (row, c) of
// pass p, so that the two 1 KB fragments of one K-step are adjacent.
RWKV_DEV size_t frag_pos2(int row, int c, int C, int p) {
  return (((((size_t)(row >> 4) * (C >> 5) + (c >> 5)) * 2 + p) * 64 + (row & 15) + 16 * ((c & 31) >> 3)) << 3) +
         (c & 7);
}

// An fp32 value as an fp16 pair: hi = fp16(v) and lo' = fp16((v - hi)·2^11)
// (v - hi is exact in fp32, and the scale keeps lo' out of fp16's subnormal
// range wherever hi is normal), so hi + 2^-11·lo' carries v to about 22 bits.
// Valid for |v| < 65504 (fp16's range).
constexpr float kLoScale = 2048.f, kLoUnscale = 1.f / 2048.f;
RWKV_DEV void split_f16(float v, f16& hi, f16& lo) {
  hi = (f16)v;
  lo = (f16)((v - (float)hi) * kLoScale);
}

// Raw buffer loads over the byte range [base, base + bytes): an offset at or
// past the end reads 0, so rows past the end need neither a clamp nor a
// select (a select on a loaded value can be turned into a branch around the
// load, which then waits for it at once).  kOOB is past every range.
constexpr unsigned kOOB = 0xFFFFFFF0u;
RWKV_DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
RWKV_DEV u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
RWKV_DEV unsigned buf_load4(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
RWKV_DEV unsigned short buf_load2(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// One 32x32 MFMA step per dtype: D(32x32,f32) += A(32xKS) * B(KSx32).
// Operand lane layout (all three): lane l feeds row/column (l % 32) with KV
// consecutive k values starting at (l / 32) * KV.  The 16 accumulators of
// lane l hold column (l % 32), rows 8*(v/4) + 4*(l/32) + (v%4), v = 0..15.
template <typename T> struct Mma32;
template <> struct Mma32<f16> {
  static constexpr int KS = 16, KV = 8;
  typedef f16x8 frag;
  typedef f32x16 acc;
  static constexpr int ACC = 16;
  static RWKV_DEV f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma32<bf16> {
  static constexpr int KS = 16, KV = 8;
  typedef bf16x8 frag;
  typedef f32x16 acc;
  static constexpr int ACC = 16;
  static RWKV_DEV f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma32<float> {
  static constexpr int KS = 2, KV = 1;
  typedef float frag;
  typedef f32x16 acc;
  static constexpr int ACC = 16;
  static RWKV_DEV f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

// 16x16 MFMA step: D(16x16,f32) += A(16xKS) * B(KSx16).  Lane l feeds row /
// column (l % 16) with KV consecutive k values from (l / 16) * KV; its 4
// accumulators hold column (l % 16), rows 4 * (l / 16) + v.
template <typename T> struct Mma16;
template <> struct Mma16<f16> {
  static constexpr int KS = 32, KV = 8;
  typedef f16x8 frag;
  typedef f32x4 acc;
  static constexpr int ACC = 4;
  static RWKV_DEV f32x4 run(frag a, frag b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <> struct Mma16<bf16> {
  static constexpr int KS = 32, KV = 8;
  typedef bf16x8 frag;
  typedef f32x4 acc;
  static constexpr int ACC = 4;
  static RWKV_DEV f32x4 run(frag a, frag b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};
template <> struct Mma16<float> {
  static constexpr int KS = 4, KV = 1;
  typedef float frag;
  typedef f32x4 acc;
  static constexpr int ACC = 4;
  static RWKV_DEV f32x4 run(frag a, frag b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
};

RWKV_DEV int acc_row(int v, int lane) { return ((v >> 2) << 3) + ((lane >> 5) << 2) + (v & 3); }

// MFMA shape selector: MN = 32 -> 32x32 blocks, MN = 16 -> 16x16 blocks.
// Lane l feeds row / column (l % MN) with KV k values from (l / MN) * KV;
// accumulator v of lane l holds column (l % MN) and row acc_row_n<MN>(v, l).
template <typename T, int MN> struct MmaSel;
template <typename T> struct MmaSel<T, 32> { typedef Mma32<T> type; };
template <typename T> struct MmaSel<T, 16> { typedef Mma16<T> type; };
template <int MN> RWKV_DEV int acc_row_n(int v, int lane) {
  if constexpr (MN == 32) return acc_row(v, lane);
  else return ((lane >> 4) << 2) + v;
}

#define RWKV_DISPATCH_DTYPE(dt, T, ...)                 \
  switch (dt) {                                         \
    case 0: { typedef float T; __VA_ARGS__; } break;    \
    case 1: { typedef f16 T; __VA_ARGS__; } break;      \
    case 2: { typedef bf16 T; __VA_ARGS__; } break;     \
    default: return hipErrorInvalidValue;               \
  }
