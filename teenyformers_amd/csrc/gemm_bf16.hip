// bf16 GEMM on the gfx950 matrix cores: y[M, N] = x[M, K] . w[N, K]^T with
// fp32 accumulation, y rounded to bf16 (nearest even).  This is the Linear
// behind sym_linear (reference src/layers/mod.rs:54-58: external teeny-core
// Linear, W [out, in], no bias) at prompt sizes; decode-step sizes (M <= 16)
// run the weight-streaming kernels of linear_bf16.hip instead.
//
// Both operands are K-contiguous rows, which is exactly the operand form of
// v_mfma_f32_32x32x16_bf16 (each lane holds 8 consecutive k of one row), so
// neither needs a transpose.
//
// One workgroup of 8 wavefronts (two per SIMD) computes a 256 x 256 tile of
// y; wavefront (wm, wn) owns rows 128 wm .. +128 and columns 64 wn .. +64,
// 4 x 2 accumulators of 32 x 32 (128 VGPRs).  K advances 64 at a time: the
// x and w tiles (256 x 64 each, 32 KiB) stream global -> LDS by
// buffer_load ... lds one tile ahead into two buffers (128 KiB), and each
// 16-k step reads the wavefront's 4 x-fragments and 2 w-fragments
// (ds_read_b128) two steps ahead of its 8 products, across tile boundaries
// (three register sets).  LDS rows are 128 bytes (two per 256-byte line);
// 16-byte chunk c of row r sits at position c ^ ((r >> 1) & 7) of its row,
// so the 16 rows a 16-lane read pass touches (one chunk each) hit 16
// distinct bank groups.  Measured at the Llama shapes (M 8192): 0.9-1.3
// PFLOP/s, 0.78-0.83x the library GEMM (hipBLASLt), whose kernels issue
// fewer LDS bytes per product (one wavefront per SIMD, larger wavefront
// tiles).
//
// Tile order: workgroup ids are remapped so that each XCD (own L2) takes a
// contiguous share of tiles, walked in groups of 4 tile-rows, column by
// column: the ~32 workgroups resident on an XCD share 4 x-row tiles and 8
// w-row tiles.
//
// Rows past M or N lie outside the operands' buffer ranges and load as
// zeros (their outputs are not stored); K must be a multiple of 64 and N of
// 64 (checked by the host).
#include "cdna4.h"

#include <numeric>
#include <type_traits>

namespace {


// LDS byte offset of 16-byte chunk c of tile row r (rows of BK bf16):
// BK = 64: 128-byte rows, two per line, c ^= (r >> 1) & 7;
// BK = 32: 64-byte rows, four per line, c ^= (r >> 2) & 3.
template <int BK>
DEVI int gpos(int r, int c) {
  if constexpr (BK == 64) return r * 128 + ((c ^ ((r >> 1) & 7)) << 4);
  else return r * 64 + ((c ^ ((r >> 2) & 3)) << 4);
}

// BM x BN: the workgroup's tile of y; BK: K per LDS tile; NS: tiles in
// flight (LDS buffers); WAVES: wavefronts per workgroup, WGM of them along M
// (WAVES / WGM along N); GROUP_M: tile-rows per group of the tile order; RA:
// 16-k steps of fragment read-ahead; IL: the refill's loads are issued IL at a
// time between the products of the step that issues them (0: all at once).
// SWIGLU: w is a fused gate_up weight [2N, K] (gate rows, then up rows) and
// y[M, N] = silu(g) * u with g = bf16(x w_gate^T), u = bf16(x w_up^T): the
// workgroup's BN W rows are BN/2 gate rows and the matching BN/2 up rows,
// each wavefront's two 32-column blocks a gate block and its up block, so
// the epilogue holds both factors of every output in one lane.
template <int BM, int BN, int BK, int NS, int WAVES, int WGM, int GROUP_M, int RA, int IL = 0,
          bool SWIGLU = false>
__device__ __forceinline__ void gemm_bf16_nt(const bf16* __restrict__ x, const bf16* __restrict__ w,
                             bf16* __restrict__ y, int M, int N, int K, int tiles_m,
                             int tiles_n) {
  constexpr int XTILE = BM * BK * 2, WTILE = BN * BK * 2;  // bytes per operand tile
  constexpr int NT = 64 * WAVES;                // threads
  constexpr int LPX = XTILE / (NT * 16);        // 16-byte DMA loads per thread, x tile
  constexpr int LPW = WTILE / (NT * 16);        // ... w tile
  constexpr int STEPS = BK / 16;                // 16-k steps per tile
  static_assert(RA <= STEPS, "fragments are read at most one tile ahead");
  constexpr int WGN = WAVES / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN;   // wavefront tile
  constexpr int I = WM / 32, J = WN / 32;        // 32 x 32 blocks per wavefront
  constexpr int CPR = BK / 8;                    // 16-byte chunks per row
  // one LDS object: with the x and w tiles in separate __shared__ arrays the
  // compiler waited for every LDS DMA in flight before each fragment read
  struct __attribute__((aligned(16))) Smem {
    char x[NS][XTILE];
    char w[NS][WTILE];
  };
  __shared__ Smem sm;
  auto& smx = sm.x;
  auto& smw = sm.w;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int wm = wave / WGN, wn = wave % WGN;

  // ---- tile of this workgroup ----------------------------------------------
  const int total = tiles_m * tiles_n;
  const int id = xcd_remap(blockIdx.x, total);
  const int per_group = GROUP_M * tiles_n;
  const int grp = id / per_group;
  const int first_m = grp * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int in_grp = id - grp * per_group;
  const int tm = first_m + in_grp % gm, tn = in_grp / gm;
  const int m0 = tm * BM;
  const int n0 = tn * (SWIGLU ? BN / 2 : BN);  // first output column
  static_assert(!SWIGLU || J == 2, "a gate block and an up block per wavefront");

  // ---- DMA sources: slot P = j * NT + tid (16 bytes) of a tile holds the
  //      chunk of row r = P / CPR whose position gpos gives.  Load j of a
  //      thread is its load 0 shifted by j * NT / CPR rows (a multiple of 32,
  //      which keeps the swizzle), so only that row offset changes, and it
  //      is uniform.  Rows past M or N fall outside the buffer range: the
  //      loads return zeros (no access), and they only feed outputs that
  //      are not stored. ---------------------------------------------------
  static_assert((NT / CPR) % 32 == 0, "row step of the DMA loads keeps the swizzle");
  const int rows_x = min(BM, M - m0);
  const int rows_w = SWIGLU ? min(BN / 2, N - n0) : min(BN, N - n0);
  const auto xr = make_rsrc(x + (long)m0 * K, rows_x * K * 2);
  const auto wr = make_rsrc(w + (long)n0 * K, rows_w * K * 2);
  // SWIGLU: the tile's second half of W rows, the up rows of the same features
  const auto wu = make_rsrc(w + ((long)N + n0) * K, rows_w * K * 2);
  constexpr int WH = LPW / 2;  // W loads per half tile
  uint32_t src0;
  {
    const int r = tid / CPR;
    const int c = (gpos<BK>(r, tid % CPR) - r * BK * 2) >> 4;  // the swizzle is an involution
    src0 = (uint32_t)(r * K * 2 + c * 16);
  }
  const int jstride = (NT / CPR) * K * 2;  // bytes between load j and j + 1
  auto load = [&](int kt, int buf) {
    const int soff = __builtin_amdgcn_readfirstlane(kt * BK * 2);
#pragma unroll
    for (int j = 0; j < LPX; ++j)
      dma16(xr, smx[buf] + j * NT * 16 + wave * 1024, src0, soff + j * jstride);
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      if (SWIGLU && j >= WH)
        dma16(wu, smw[buf] + j * NT * 16 + wave * 1024, src0, soff + (j - WH) * jstride);
      else
        dma16(wr, smw[buf] + j * NT * 16 + wave * 1024, src0, soff + j * jstride);
    }
  };

  // ---- fragment read offsets: lane reads row (block + l32), chunk 2 kk + g;
  //      the swizzle repeats every 32 rows, so block i adds i * 32 rows (an
  //      immediate offset) to block 0's address ---------------------------
  constexpr int ROWB = BK * 2;
  int xoff[STEPS], woff[STEPS];
#pragma unroll
  for (int kk = 0; kk < STEPS; ++kk) {
    xoff[kk] = gpos<BK>(wm * WM + l32, 2 * kk + g);
    woff[kk] = gpos<BK>(wn * (SWIGLU ? WN / 2 : WN) + l32, 2 * kk + g);
  }
  // W block j starts JROWS rows after block 0: the next 32 rows, or with
  // SWIGLU the up rows of the gate block's features (half a tile on)
  constexpr int JROWS = SWIGLU ? BN / 2 : 32;

  f32x16 acc[I][J];
#pragma unroll
  for (int i = 0; i < I; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j) acc[i][j] = f32x16{};

  const int nk = K / BK;
  // Fragments in NSET = RA + 1 register sets: 16-k step s (counted across
  // tiles) uses set s % NSET while the reads of step s + RA land in the
  // others.  Step STEPS - RA of a tile, the first to read from the next
  // tile, waits for that tile and the barrier, then refills the buffer just
  // finished with the tile NS ahead; so neither read latency nor the DMA
  // issue sits between tiles.
  constexpr int NSET = RA + 1;
  u32x4 xa[NSET][I], wb[NSET][J];
  auto rd = [&](const char* xs, const char* ws, int kk, int set) {
#pragma unroll
    for (int i = 0; i < I; ++i)
      xa[set][i] = *reinterpret_cast<const u32x4*>(xs + xoff[kk] + i * 32 * ROWB);
#pragma unroll
    for (int j = 0; j < J; ++j)
      wb[set][j] = *reinterpret_cast<const u32x4*>(ws + woff[kk] + j * JROWS * ROWB);
  };
  // y^T blocks: w rows are the A operand (the 32 rows of a block), x rows
  // the B operand (lane = x row)
  auto mm = [&](int set) {
#pragma unroll
    for (int i = 0; i < I; ++i)
#pragma unroll
      for (int j = 0; j < J; ++j)
        acc[i][j] = mfma32(as_bf16x8(wb[set][j]), as_bf16x8(xa[set][i]), acc[i][j]);
  };
  // tile t in LDS buffer CUR, its step 0 in register set S0
  auto body = [&](int t, auto CUR, auto S0) {
    constexpr int cur = decltype(CUR)::value, nxt = (cur + 1) % NS;
    constexpr int s0 = decltype(S0)::value;
#pragma unroll
    for (int kk = 0; kk < STEPS; ++kk) {
      if (kk == STEPS - RA) {
        // unconditional (a branch here made the compiler wait for the
        // reads below before the products): past the last tile the refill
        // re-reads tile nk - 1 and the reads fetch unused fragments
        __builtin_amdgcn_s_waitcnt(kVmWaitLgkm0<(NS - 2) * (LPX + LPW)>());  // tile t+1; our reads of t
        barrier_only();  // everyone's tile t+1 has landed; buffer cur is free
        load(min(t + NS, nk - 1), cur);
      }
      const int rs = kk + RA;  // each step: the reads RA steps ahead first, then products
      if (rs < STEPS) rd(smx[cur], smw[cur], rs, (s0 + rs) % NSET);
      else rd(smx[nxt], smw[nxt], rs - STEPS, (s0 + rs) % NSET);
      mm((s0 + kk) % NSET);
      sched_group(kDsRead, I + J);
      if (IL && kk == STEPS - RA) {
        // the refill's loads between the products, IL at a time
#pragma unroll
        for (int q = 0; q < I * J; ++q) {
          sched_group(kMfma, 1);
          if (q * IL < LPX + LPW) sched_group(kVmemRead, IL);
        }
      } else {
        sched_group(kMfma, I * J);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

#pragma unroll
  for (int s = 0; s < NS; ++s) load(min(s, nk - 1), s);
  __builtin_amdgcn_s_waitcnt(kVmWaitLgkm0<(NS - 1) * (LPX + LPW)>());  // tile 0
  barrier_only();
#pragma unroll
  for (int s = 0; s < RA; ++s) rd(smx[0], smw[0], s, s);
  // buffers repeat every NS tiles, register sets every NSET / gcd(STEPS,
  // NSET): unrolled over both, every LDS and register index is a constant
  constexpr int SP = NSET / std::gcd(STEPS, NSET);
  constexpr int PERIOD = NS * SP / std::gcd(NS, SP);
  for (int kt = 0; kt < nk; kt += PERIOD) {
    unroll_tiles<0, PERIOD>([&](auto TI) {
      constexpr int ti = decltype(TI)::value;
      if (kt + ti < nk)
        body(kt + ti, std::integral_constant<int, ti % NS>{},
             std::integral_constant<int, (ti * STEPS) % NSET>{});
    });
  }

  // the refills issued past the last tile land before the workgroup's LDS
  // is released
  __builtin_amdgcn_s_waitcnt(kVmWait<0>());
  // ---- y: lane = row m (l32 of each 32-row block), registers 4q..4q+3 are
  //      columns 8q + 4g .. +3 of the 32-column block ----------------------
#pragma unroll
  for (int i = 0; i < I; ++i) {
    const int m = m0 + wm * WM + i * 32 + l32;
    if (m >= M) continue;
    bf16* yr = y + (long)m * N;
    if constexpr (SWIGLU) {
      // the unfused path's arithmetic: both products rounded to bf16, then
      // silu(g) * u in fp32 and one rounding
      const int nb = n0 + wn * (WN / 2);
      if (nb >= N) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gt = bf2f(f2bf(acc[i][0][4 * q + e]));
          const float up = bf2f(f2bf(acc[i][1][4 * q + e]));
          o[e] = gt * (1.0f / (1.0f + expf(-gt))) * up;
        }
        *reinterpret_cast<u32x2*>(yr + nb + 8 * q + 4 * g) =
            u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
      }
      continue;
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int nb = n0 + wn * WN + j * 32;
      if (nb >= N) continue;  // N is a multiple of 64: whole 32-column blocks
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = nb + 8 * q + 4 * g;
        *reinterpret_cast<u32x2*>(yr + n) =
            u32x2{pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                  pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
      }
    }
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(512) void teeny_gemm_bf16_nt(
    const bf16* x, const bf16* w, bf16* y, int M, int N, int K, int tiles_m, int tiles_n) {
  gemm_bf16_nt<256, 256, 64, 2, 8, 2, 4, 2, 1>(x, w, y, M, N, K, tiles_m, tiles_n);
}

// y[M, F] = silu(x w[:F]^T) * (x w[F:]^T) for w = [gate; up] of shape [2F, K];
// tiles of 256 rows x 128 features
extern "C" __global__ __launch_bounds__(512) void teeny_gemm_swiglu_bf16_nt(
    const bf16* x, const bf16* w, bf16* y, int M, int F, int K, int tiles_m, int tiles_n) {
  gemm_bf16_nt<256, 256, 64, 2, 8, 2, 4, 2, 1, true>(x, w, y, M, F, K, tiles_m, tiles_n);
}
