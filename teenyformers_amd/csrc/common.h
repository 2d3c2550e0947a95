// Shared device-side helpers for the gfx950 (CDNA4) kernels.
//
// Every kernel is `extern "C" __global__` so the host library can look it up
// by name in the code object with hipModuleGetFunction.  Storage types are
// fp32 (`float`) and bf16 (`__bf16`, bit-compatible with the IEEE upper half
// of an fp32); arithmetic is always fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define DEVI __device__ __forceinline__

// MI355X: 8 accelerator complex dies (XCDs), each with its own L2.  The
// dispatcher hands consecutive workgroup ids to XCDs round-robin.
#define TEENY_NUM_XCD 8

DEVI float bf2f(bf16 x) { return (float)x; }
DEVI bf16 f2bf(float x) { return (bf16)x; }  // round to nearest even

DEVI uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
  return __builtin_bit_cast(uint32_t, v);
}

// Low / high bf16 of a packed pair, widened to fp32.
DEVI float bf16lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
DEVI float bf16hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// RoPE of interleaved pairs (src/kernels/rope.rs:57-97, 86-88): pair k of a
// row at position pos turns by theta = fp32(pos) * fp32(exp_f64(fp32(k) * c))
// with c = (-2 ln_base) / head_dim in fp32.  Every kernel that rotates takes
// its (cos, sin) from rope_cos_sin and rotates with rope_rotate, so that the
// same row at the same position gets the same bits in each of them.
DEVI float rope_c(float ln_base, int head_dim) { return (-2.0f * ln_base) / (float)head_dim; }
DEVI void rope_cos_sin(int pos, int k, float c, float& cn, float& sn) {
  const float inv = (float)exp((double)((float)k * c));
  sincosf((float)pos * inv, &sn, &cn);
}
// (x0, x1) -> (x0 cos - x1 sin, x0 sin + x1 cos): the second product of each
// rounded, the first fused with the sum
DEVI void rope_rotate(float x0, float x1, float cn, float sn, float& o0, float& o1) {
  o0 = __builtin_fmaf(x0, cn, -(x1 * sn));
  o1 = __builtin_fmaf(x0, sn, x1 * cn);
}

// Generic element load/store with fp32 arithmetic.
template <typename T> DEVI float ld(const T* p) { return (float)*p; }
template <typename T> DEVI void st(T* p, float v) { *p = (T)v; }

// 16-byte vector of storage elements (8 x bf16 or 4 x fp32) converted to fp32.
template <typename T> struct Vec16;
template <> struct Vec16<float> {
  static constexpr int N = 4;
  DEVI static void load(const float* p, float* out) {
    f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = v[i];
  }
  DEVI static void store(float* p, const float* in) {
    f32x4 v = {in[0], in[1], in[2], in[3]};
    *reinterpret_cast<f32x4*>(p) = v;
  }
};
template <> struct Vec16<bf16> {
  static constexpr int N = 8;
  DEVI static void load(const bf16* p, float* out) {
    u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = bf16lo(v[i]);
      out[2 * i + 1] = bf16hi(v[i]);
    }
  }
  DEVI static void store(bf16* p, const float* in) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(in[2 * i], in[2 * i + 1]);
    *reinterpret_cast<u32x4*>(p) = v;
  }
};

// VEC consecutive values of a sum of n fp32 partial slabs (slab s at
// part + s * stride), added in slab order and rounded to T: what a product
// split over K gives once its parts are summed and stored in T.  CH chunks
// at part + off[c] are summed at once.  The loads of a group of U slabs are
// all issued before the first add (unconditionally: slabs past n re-read slab
// n - 1 and are not added), so a call waits for memory once per group.
template <typename T, int VEC, int CH>
DEVI void ld_parts(const float* __restrict__ part, long stride, int n, float (*out)[VEC],
                   const int* off) {
  static_assert(VEC % 4 == 0, "16-byte loads");
  constexpr int U = CH >= 4 ? 4 : 8;  // slabs in flight together
  float acc[CH][VEC];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[c][j] = 0.0f;
  for (int s = 0; s < n; s += U) {
    f32x4 v[U][CH][VEC / 4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float* src = part + min(s + u, n - 1) * stride;
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int j = 0; j < VEC / 4; ++j)
          v[u][c][j] = *reinterpret_cast<const f32x4*>(src + off[c] + 4 * j);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (s + u < n)
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
          for (int j = 0; j < VEC / 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[c][4 * j + i] += v[u][c][j][i];
  }
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int j = 0; j < VEC; ++j) out[c][j] = (float)(T)acc[c][j];
}
template <typename T, int VEC>
DEVI void ld_parts(const float* __restrict__ part, long stride, int n, float* out) {
  const int off[1] = {0};
  ld_parts<T, VEC, 1>(part, stride, n, reinterpret_cast<float(*)[VEC]>(out), off);
}

// Wavefront (64-lane) reductions through DPP/permute, all lanes get the result.
DEVI float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
DEVI float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Order of the (head, block) work items behind the remapped ids: heads in
// groups of G, the blocks of a group interleaved heaviest first.  Causal
// blocks differ in cost by up to n_blocks x; taken head by head (heaviest
// first), the heaviest blocks of an XCD's last head started last and
// finished ~5 % after the rest at 32 blocks per head.  Interleaving G heads
// starts the next group's heavy blocks while the previous group's light
// ones run, keeping workgroups in flight on a few heads' K/V.  A schedule
// model of an XCD's slots (workgroup time = fixed + per-tile cost, both
// measured) puts the forward at 1.06 x the ideal makespan with pairs and
// 1.02 x with groups of 4 (B8 H32 S4096, 96 slots), 1.25 x and 1.11 x at
// B16 Hq32 Hkv8 S512, with the same heads in flight (measured: 1.01 x and
// 1.06 x); the backward kernels' 64 slots per XCD reach the ideal with
// pairs.  G is the largest power of
// two up to GMAX for which every XCD's contiguous share of ids holds whole
// groups (n_heads a multiple of 8 G): a group split between two XCDs would
// hand one of them all the heavy blocks.  rank 0 is a head's heaviest
// block.  Bijective on [0, n_heads * n_blocks).
template <int GMAX = 2>
DEVI void pair_order(int id, int n_blocks, int n_heads, int& head, int& rank) {
  int gsz = 1;
  if (GMAX >= 4 && n_heads % (4 * TEENY_NUM_XCD) == 0) gsz = 4;
  else if (GMAX >= 2 && n_heads % (2 * TEENY_NUM_XCD) == 0) gsz = 2;
  const int grp = id / (gsz * n_blocks);
  const int r = id - grp * gsz * n_blocks;
  head = gsz * grp + r % gsz;
  rank = r / gsz;
}

// Remap a linear workgroup id so that consecutive ids in the returned space
// land on the same XCD (the hardware deals ids round-robin across XCDs).
// Bijective for any total.
DEVI int xcd_remap(int id, int total) {
  int xcd = id % TEENY_NUM_XCD;
  int local = id / TEENY_NUM_XCD;
  int q = total / TEENY_NUM_XCD, r = total % TEENY_NUM_XCD;
  return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}
