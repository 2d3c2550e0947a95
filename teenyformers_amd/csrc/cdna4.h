// gfx950 building blocks shared by the bf16 attention kernels: the 32x32x16
// bf16 MFMA, LDS transpose reads, buffer-to-LDS DMA, tile swizzles and a few
// single-instruction helpers.
#pragma once
#include "common.h"

#include <type_traits>

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

DEVI float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
DEVI bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
DEVI f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// max of three floats (one v_max3_f32).  A builtin, not inline asm: the
// compiler must see the instruction to keep the wait states that an MFMA
// result read right after the product, or an MFMA operand register
// overwritten right after its issue, requires.  Files that take their
// inputs from MFMA results are compiled with -fno-honor-nans, so no
// canonicalising v_max is added per operand (scores are never NaN).
DEVI float max3(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }
// the value held by lane l ^ 32 (v_permlane32_swap)
DEVI float other_half(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x),
                                            __builtin_bit_cast(unsigned, x), false, false);
  // lanes < 32 see (x[l], x[l+32]), lanes >= 32 see (x[l-32], x[l])
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}
// acc + lo + hi of a packed bf16 pair (v_dot2c_f32_bf16 against (1, 1))
DEVI float add_bf16x2(uint32_t w, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, w),
                                         __builtin_bit_cast(b2, 0x3f803f80u), acc, false);
}

// Instruction classes of __builtin_amdgcn_sched_group_barrier: the machine
// scheduler fills the groups in the order they are declared.
constexpr int kMfma = 0x008, kVmemRead = 0x020, kDsRead = 0x100;
#define sched_group(mask, n) __builtin_amdgcn_sched_group_barrier((mask), (n), 0)
// Keeps the computation of x above this point: values used only in the next
// loop iteration would otherwise be sunk below the barrier that ends one,
// out of the block they are scheduled in.
template <typename T> DEVI void pin(T& x) { asm volatile("" : "+v"(x)); }

// ds_read_b64_tr_b16: within each 16-lane group, output lane i receives
// element (i % 4) of the 8-byte chunks addressed by lanes i/4, i/4+4, i/4+8
// and i/4+12 (measured on gfx950): lanes addressing a 4-row x 16-column block
// of a row-major tile receive it transposed, one column per lane.
DEVI u32x2 lds_read_tr(const char* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

// Raw buffer descriptor (stride 0, num_records in bytes) over [base, +bytes).
DEVI __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
// buffer_load_dwordx4 ... lds: 16 bytes per lane from buffer offset
// soff + voff into LDS at lds + 16 * lane.  A MUBUF load, not FLAT: with FLAT
// LDS loads in flight the compiler waits for every LDS read to drain.
DEVI void dma16(__amdgpu_buffer_rsrc_t r, char* lds, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voff, soff, 0, 0);
}

// Tiles are stored unpadded: 16-byte chunk L = row * (D/8) + column chunk,
// XOR-swizzled within each 256-byte line (64 banks x 4 bytes); the position
// of L is swz(L) (an involution).
//   SWZ_ROW  (read by rows, 16 bytes per lane): position ^= line % 16.
//   SWZ_DUAL (read by rows and by 4-row transpose reads): position ^= a
//            bijection of the row's low four bits whose top two bits are the
//            row's lowest two, so 16 consecutive rows of a row read and the
//            4 rows x 4 chunks of a transpose-read half-wave touch distinct
//            banks.  D = 128: x = (r&3)<<2 | (r>>2)&3 (one row per line);
//            D = 64: two rows per line, x = (line&1)<<2 | (line>>1)&3.
// Both repeat every 16 rows for D in {64, 128} and every 256 chunks.
enum Swz { SWZ_ROW, SWZ_DUAL };
template <Swz S, int D>
DEVI int swz(int L) {
  const int line = L >> 4, pos = L & 15;
  int x;
  if (S == SWZ_ROW) x = line & 15;
  else if (D == 128) x = ((line & 3) << 2) | ((line >> 2) & 3);
  else x = ((line & 1) << 2) | ((line >> 1) & 3);
  return (line << 4) | (pos ^ x);
}

// s_waitcnt immediate for vmcnt(n) alone (expcnt, lgkmcnt fields at their
// maximum: not waited for); n < 64
template <int n>
constexpr int kVmWait() {
  static_assert(n < 64, "vmcnt has 6 bits");
  return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8);
}
// ... and lgkmcnt(0)
template <int n>
constexpr int kVmWaitLgkm0() {
  return kVmWait<n>() & ~(15 << 8);
}

// s_barrier alone: __syncthreads() also waits for every memory operation in
// flight (vmcnt(0)), which would wait for the tiles loading further ahead;
// the caller waits for exactly what the barrier publishes.  The memory
// clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// f(integral_constant<T>) for T = B .. E-1
template <int B, int E, typename F>
__device__ __forceinline__ void unroll_tiles(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    unroll_tiles<B + 1, E>(f);
  }
}

// Stores a wavefront's 32-row output tile whose lane l holds, per MFMA
// d-tile t and j = 0..3, the 4 values of row l % 32 at d = 32 t + 8 j +
// 4 (l / 32) .. +3 (the 32x32 accumulator layout): through the wavefront's
// LDS area `tile` (32 x D values of GT; the caller has made it free), the
// 16-byte chunk c of row r placed at chunk c ^ (r % 16) of the row, then
// read back and stored a whole row per D sizeof(GT) / 16 lanes.  A store
// straight from the accumulators writes 32 scattered pieces per
// instruction, which held a workgroup ~2 us longer on its CU.  vals(t, j)
// returns the lane's 4 values; rows r < rows_valid are stored at
// dst + r * D.  The lane-dependent offsets are formed here, behind an empty
// asm, so they are not hoisted into (and kept live through) a caller's loop.
template <int D, typename GT, typename F>
DEVI void store_tile_rows(char* tile, GT* dst, int rows_valid, F&& vals) {
  constexpr int ES = (int)sizeof(GT);
  constexpr int RB = D * ES;            // bytes per row
  constexpr int CPR = RB / 16;          // 16-byte chunks per row
  constexpr int MASK = (CPR < 16 ? CPR : 16) - 1;
  constexpr int RPI = 64 / CPR;         // rows per store
  static_assert(ES == 2 || ES == 4, "bf16 or fp32 rows");
  const int ln = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int lr = ln & 31, hg = ln >> 5;
  // write of (t, j): bf16: chunk 4 t + j, bytes 8 hg of it; fp32: chunk
  // 8 t + 2 j + hg, all 16 bytes
  int wa = lr * RB + (ES == 2 ? ((lr & MASK) << 4) + 8 * hg : (((lr & MASK) ^ hg) << 4));
  int ra = (ln / CPR) * RB + (((ln % CPR) ^ ((ln / CPR) & MASK)) << 4);
  int sa = (ln / CPR) * D + (ln % CPR) * (16 / ES);
  asm volatile("" : "+v"(wa), "+v"(ra), "+v"(sa));
#pragma unroll
  for (int t = 0; t < D / 32; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 x = vals(t, j);
      if constexpr (ES == 2)
        *reinterpret_cast<u32x2*>(tile + (wa ^ ((4 * t + j) << 4))) =
            u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
      else
        *reinterpret_cast<f32x4*>(tile + (wa ^ ((8 * t + 2 * j) << 4))) = x;
    }
#pragma unroll
  for (int kk = 0; kk < 32 / RPI; ++kk) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(
        tile + (ra ^ (((kk * RPI) & MASK) << 4)) + kk * RPI * RB);
    if (kk * RPI + ln / CPR < rows_valid)
      *reinterpret_cast<u32x4*>(dst + kk * RPI * D + sa) = v;
  }
}
