// gemm_fp8.hip -- prefill FP8 x FP8 GEMM on the gfx950 matrix cores.
//
// Y[m, n] = alpha * ((a_m * s_n) * sum_k e4m3(XA[m, k]) * e4m3(Q[n, k])),
// XA row-major [M][ldxq] (per-token scales a_m), Q in the FP8 wave-tile
// layout of layout.hpp (per-row scales s_n), fp32 accumulation.
//
// Two kernels: an LDS-pipelined one for M >= 128 with K % 128 == 0 and
// aligned activation rows (the prefill shapes), and a direct-from-L2 one that
// loads operands straight from global memory in MFMA lane order for every
// other shape.
#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <set>
#include <utility>

#include "device_common.hpp"
#include "kernels.hpp"

#include "weight.hpp"

namespace ullm {
namespace {

typedef long i64;

__device__ __forceinline__ f32x4 mfma_fp8(i64 a, i64 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a, b, c, 0, 0, 0);
}

// 16 activation bytes of row m at k0 (zero beyond M or K).
__device__ __forceinline__ u32x4 load_xq16(const uint8_t *__restrict__ row,
                                           bool valid, uint32_t k0, uint32_t K,
                                           bool vec) {
  u32x4 r = {0u, 0u, 0u, 0u};
  if (valid) {
    if (vec && k0 + 16 <= K) {
      r = *reinterpret_cast<const u32x4 *>(row + k0);
    } else {
      uint32_t b[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t v = (k0 + i < K) ? row[k0 + i] : 0u;
        b[i / 4] |= v << (8 * (i % 4));
      }
      r = u32x4{b[0], b[1], b[2], b[3]};
    }
  }
  return r;
}

struct GemmArgs {
  const uint8_t *xq;
  const float *xs;
  const uint8_t *tiles;
  const float *scales;
  void *y;
  uint64_t ldxq, ldy;
  uint32_t m, n, k, units;
  float alpha;
  bool y_f32;
  bool y_vec;  // bf16 rows 16-byte aligned: coalesced epilogue stores
  Epilogue epi;
  // Split K (ping-pong blocks on grids of few tiles): K parts per tile, a
  // counter per tile (zero on entry, left zero) and the fp32 partial sums.
  uint32_t ksplit;
  uint32_t *cnt;
  float *part;
  uint32_t part_bytes;
};

// 256 threads, block tile 64 (m) x 64 (n); wave (wm, wn) owns 32 x 32.
template <uint32_t EPI>
__global__ __launch_bounds__(256) void fp8_gemm_direct_kernel(GemmArgs a,
                                                              bool vec) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const uint32_t m0 = blockIdx.y * 64 + (wave / 2) * 32;
  const uint32_t T0 = blockIdx.x * 4 + (wave % 2) * 2;  // 16-row stripes
  const uint32_t stripes = (a.n + 15) / 16;
  const uint8_t *rows[2];
  bool valid[2];
  for (int i = 0; i < 2; ++i) {
    const uint32_t m = m0 + i * 16 + lane % 16;
    valid[i] = m < a.m;
    rows[i] = a.xq + uint64_t(valid[i] ? m : 0) * a.ldxq;
  }
  f32x4 acc[2][2];
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint32_t kl = 16 * (lane / 16);
  for (uint32_t u = 0; u < a.units; ++u) {
    u32x4 bw[2];
    for (int j = 0; j < 2; ++j) {
      const uint32_t T = T0 + j < stripes ? T0 + j : stripes - 1;
      bw[j] = *reinterpret_cast<const u32x4 *>(
          a.tiles + (uint64_t(T) * a.units + u) * 1024 + lane * 16);
    }
    for (int i = 0; i < 2; ++i) {
      const u32x4 av = load_xq16(rows[i], valid[i], u * 64 + kl, a.k, vec);
      const i64 a0 = __builtin_bit_cast(i64, u32x2{av.x, av.y});
      const i64 a1 = __builtin_bit_cast(i64, u32x2{av.z, av.w});
      for (int j = 0; j < 2; ++j) {
        const i64 b0 = __builtin_bit_cast(i64, u32x2{bw[j].x, bw[j].y});
        const i64 b1 = __builtin_bit_cast(i64, u32x2{bw[j].z, bw[j].w});
        acc[i][j] = mfma_fp8(a0, b0, acc[i][j]);
        acc[i][j] = mfma_fp8(a1, b1, acc[i][j]);
      }
    }
  }
  for (int i = 0; i < 2; ++i) {
    for (int j = 0; j < 2; ++j) {
      const uint32_t n = (T0 + j) * 16 + lane % 16;
      for (int r = 0; r < 4; ++r) {
        const uint32_t m = m0 + i * 16 + 4 * (lane / 16) + r;
        const uint32_t mc = m < a.m ? m : a.m - 1;
        const uint32_t nc = n < stripes * 16 ? n : stripes * 16 - 1;
        const float v = a.alpha * ((a.xs[mc] * a.scales[nc]) * acc[i][j][r]);
        store_out<EPI>(a.y, a.ldy, a.y_f32, a.epi, a.n, m, n, v, m < a.m);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// LDS-pipelined kernel (v_mfma_f32_16x16x128_f8f6f4, fp8 x fp8).
//
// Block tile BM x BN x 128 (k), WM x WN waves, each wave owning a
// (BM / WM) x (BN / WN) output tile of 16 x 16 MFMA tiles.  B is staged as
// 1 KiB "wave tiles": 16 rows x 64 k in MFMA lane order (lane l = row l % 16,
// 16 bytes at k = 16 * (l / 16)), the order the weights already have in HBM.
// A (row-major activations) is staged as whole 128-byte row segments with
// swizzled chunks (layout at the copy offsets below).  A lane's 32-byte MFMA
// operand is its 16 bytes of k [0, 64) followed by those of [64, 128), for A
// and B alike, so the k pairing matches; every LDS read is a ds_read_b128
// without bank conflicts.  Global -> LDS moves are direct buffer loads into
// LDS (no registers); two stages alternate so the copies of step s + 1 run
// under the MFMAs of step s.  The 256-row blocks (8 waves) run the
// ping-pong main loop described at the loop; a 128 x 128 block fits two
// workgroups per CU but doubles the operand traffic from L2 per flop (1.37
// against 1.96 PFLOP/s for 256 x 256 before the ping-pong loop, at M=2048,
// N=28672, K=4096), so it serves only grids the large blocks leave half
// empty.  Activation rows are copied
// as whole 128-byte lines (see the A stage layout below): copying them as
// 16-row wave tiles, 64 bytes per row per copy, capped the copy pipeline at
// 8 TB/s from L2 and the kernel at 1.75 PFLOP/s.
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));

template <uint32_t BM_, uint32_t BN_, uint32_t WM_, uint32_t WN_,
          uint32_t BSTAGES_ = 2, uint32_t ASTAGES_ = 2, bool PP_ = false>
struct GemmCfg {
  static constexpr uint32_t BM = BM_, BN = BN_, BK = 128, WM = WM_, WN = WN_;
  // Ping-pong main loop: the two halves of the waves (one wave of each per
  // SIMD) alternate between reading their operands from LDS and running
  // their MFMAs, so each SIMD's matrix core works while its other wave
  // waits on LDS.
  static constexpr bool PP = PP_;
  // A (activations, L2-resident) is double-buffered; B (weights, streamed
  // from HBM) may get a third buffer so its copies run two k-steps ahead.
  static constexpr uint32_t BSTAGES = BSTAGES_;
  // A third A buffer lets the activation copies run two k-steps ahead.
  // Measured slower on MI355X in the 256 x 256 block before the ping-pong
  // loop at M=2048, N=28672, K=4096 (264-270 against 250-252 us: the copies
  // were not waiting on latency there), faster in the ping-pong 256 x 128
  // and 256 x 64 blocks, whose grids of at most a few rounds leave each CU
  // waiting on its copies (below).
  static constexpr uint32_t ASTAGES = ASTAGES_;
  // Look-ahead of one or two k-steps, up to three in the ping-pong loop.
  static_assert(ASTAGES >= 2 && BSTAGES >= 2 && ASTAGES <= (PP ? 4 : 3) &&
                    BSTAGES <= (PP ? 4 : 3),
                "k-steps of look-ahead");
  static constexpr uint32_t WAVES = WM * WN;
  static constexpr uint32_t TM = BM / WM / 16;  // 16-row m-tiles per wave
  static constexpr uint32_t TN = BN / WN / 16;  // 16-column n-tiles per wave
  static constexpr uint32_t A_TILES = BM / 16 * 2, B_TILES = BN / 16 * 2;
  static constexpr uint32_t A_BYTES = A_TILES * 1024;
  static constexpr uint32_t B_BYTES = B_TILES * 1024;
  static constexpr uint32_t STAGE_BYTES = ASTAGES * A_BYTES + BSTAGES * B_BYTES;
  // Waves issuing each operand's global -> LDS copies (CW of them).
  static constexpr uint32_t CW = PP ? WAVES / 2 : WAVES;
  static constexpr uint32_t A_COPIES = A_TILES / CW;
  // B copies per wave; when the waves do not split B evenly, the last round
  // of copies is done by the first B_TILES % CW waves only.
  static constexpr uint32_t B_COPIES = (B_TILES + CW - 1) / CW;
  static constexpr bool B_EVEN = B_TILES % CW == 0;
  static_assert(A_TILES % CW == 0, "copy split");
  // Row pitch (bf16 elements) of a wave's epilogue chunk: a row of its
  // tile, padded by 16 bytes so the rows of one LDS store land in different
  // banks.
  static constexpr uint32_t OUT_STRIDE = TN * 16 + 8;
  // bf16 output is staged one 16-row m-tile per wave at a time, past the
  // operand stages (or in A stage 1, below), so the stages the next tile's
  // first copies fill stay free.
  static constexpr uint32_t CHUNK_BYTES = 16 * OUT_STRIDE * 2;
  // The ping-pong loop runs with three B stages: waves 0-3 copy A one
  // k-step ahead, waves 4-7 copy B two k-steps ahead, each in its own read
  // phase, so the copy issue of a k-step is split over its two phases; the
  // epilogue chunks then live in A stage 1, which the next tile's first
  // copies leave alone.
  // With a third A stage (A copied two k-steps ahead too) the chunks move
  // to A stage 2: the next tile's first copies fill A stages 0 and 1.
  // Blocks whose A stage is too small for them keep the chunks past the
  // stages.
  static_assert(!PP || BSTAGES >= 3, "ping-pong: at least three B stages");
  static constexpr bool CHUNKS_IN_A = PP && WAVES * CHUNK_BYTES <= A_BYTES;
  static constexpr uint32_t CHUNK_BASE =
      CHUNKS_IN_A ? (ASTAGES - 1) * A_BYTES : STAGE_BYTES;
  // The ping-pong loop waits for a step's B copies by count (each copying
  // wave issues B_COPIES per step), so every copying wave must issue as many.
  static_assert(!PP || B_TILES % CW == 0, "B copies split evenly");
  static constexpr uint32_t LDS = STAGE_BYTES + (CHUNKS_IN_A ? 0 : WAVES * CHUNK_BYTES);
  // The short-prompt blocks load their epilogue's row and column scales at
  // the tile's start, under its first copies, instead of after the k-loop
  // (MI355X: M=64 N=4096 K=4096 11.9 against 12.5 us, M=256 N=6144 18.0
  // against 18.5, M=64 N=28672 26.1-26.3 against 26.8-27.0).  The wide
  // blocks keep the late gather: early, it measured level on the 224-, 192-
  // and 128-column blocks and slowed the 256 x 256 one from 55 to 101 us
  // (M=2048 N=8192).
  static constexpr bool EARLY_SCALES = PP && BM < 256;
  static_assert(LDS <= 160 * 1024, "gfx950 LDS per workgroup");
};

// Zero scale operands: the compiler emits the unscaled
// v_mfma_f32_16x16x128_f8f6f4 (fp8 x fp8, format code 0 for both).
__device__ __forceinline__ f32x4 mfma_fp8_k128(i32x8 a, i32x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0,
                                                          0, 0);
}

// 16 bytes per lane from a buffer resource into LDS at the wave's base
// (M0): 32-bit lane offset, scalar k-step offset, so no 64-bit per-lane
// addresses are held in registers.
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rsrc,
                                          uint32_t voff, uint32_t soff,
                                          void *lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void *)(lds_wave_base), 16,
      voff, soff, 0, 0);
}

// Cache policy of the split-K partial sums: sc0 | sc1 (system coherent).
constexpr int kScGemm = 1 | 16;

// Barrier without the fence of __syncthreads: LDS reads of this wave are
// complete (lgkmcnt 0); the caller has already waited for its copies.
__device__ __forceinline__ void gemm_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_s_barrier();
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) |
                             (0xf << 8));
}

__device__ __forceinline__ i32x8 lds_operand(const char *p) {
  const u32x4 lo = *reinterpret_cast<const u32x4 *>(p);
  const u32x4 hi = *reinterpret_cast<const u32x4 *>(p + 1024);
  const u32x8 v = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  return __builtin_bit_cast(i32x8, v);
}

// Lane exchanges through DPP (no LDS crossbar, no lgkm wait): quad_perm
// [1,0,3,2] swaps lanes across bit 0, [2,3,0,1] across bit 1, and row_ror:8
// swaps the halves of each 16-lane row (lane ^ 8).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xb1, kDppXor2 = 0x4e, kDppXor8 = 0x128;

// Four rows x one column per lane (an MFMA result) -> one row x four
// columns: within each lane quad, lane q ends with row q of the quad's four
// columns, in column order.  Two exchanges: across lane bit 1 (row pairs),
// then across lane bit 0 (single rows).
__device__ __forceinline__ f32x4 quad_transpose_f32(f32x4 v, uint32_t lane) {
  const uint32_t q = lane & 3u;
  const bool b1 = q & 2u, b0 = q & 1u;
  // Keep rows 2 b1, 2 b1 + 1 of my column c; the partner c ^ 2 sends its
  // values of those rows.
  const float k0 = b1 ? v[2] : v[0], k1 = b1 ? v[3] : v[1];
  const float s0 = b1 ? v[0] : v[2], s1 = b1 ? v[1] : v[3];
  const float g0 = dpp_f32<kDppXor2>(s0), g1 = dpp_f32<kDppXor2>(s1);
  // Keep row 2 b1 + b0 of columns c and c ^ 2; the partner c ^ 1 sends the
  // same row of columns c ^ 1 and c ^ 3.
  const float own = b0 ? k1 : k0, par = b0 ? g1 : g0;
  const float r1 = dpp_f32<kDppXor1>(b0 ? k0 : k1);
  const float r3 = dpp_f32<kDppXor1>(b0 ? g0 : g1);
  f32x4 out;
#pragma unroll
  for (uint32_t c = 0; c < 4; ++c) {
    const uint32_t d = c ^ q;  // 0: own, 1: r1, 2: par, 3: r3
    out[c] = d == 0 ? own : d == 1 ? r1 : d == 2 ? par : r3;
  }
  return out;
}

__device__ __forceinline__ u32x2 pack_bf16x4(f32x4 t) {
  return u32x2{f32x2_to_bf16x2(t[0], t[1]), f32x2_to_bf16x2(t[2], t[3])};
}

// SPLIT: the launch splits K (a.ksplit > 1, ping-pong blocks only).  A
// separate instantiation keeps the split's bookkeeping out of every other
// launch: compiled into the persistent 256 x 224 kernel as a runtime branch
// it cost 7-8 % (M=2048 N=28672 K=4096 214-216 against 199-201 us, M=4096
// N=14336 209-211 against 192-194 on one MI355X).
template <class C, uint32_t EPI, bool SPLIT>
__global__ __launch_bounds__(C::WAVES *kWave) void fp8_gemm_lds_kernel(
    GemmArgs a) {
  static_assert(!SPLIT || C::PP, "K split: ping-pong blocks only");
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t mblocks = (a.m + C::BM - 1) / C::BM;
  const uint32_t nblocks = (a.n + C::BN - 1) / C::BN;
  // A persistent grid walks tiles id = blockIdx.x + r * gridDim.x.  Tile ids
  // are dispatched round-robin over the 8 XCDs; when the tile count divides
  // evenly each XCD gets a contiguous range of tiles, so the workgroups
  // sharing one L2 also share operand tiles, and with a grid that is a
  // multiple of 8 every id of one workgroup stays on its XCD.
  // Work items: (tile, K part); without a split one per tile.
  const uint32_t ksplit = SPLIT ? a.ksplit : 1u;
  const uint32_t total = mblocks * nblocks * ksplit;
  const uint32_t stripes = (a.n + 15) / 16;
  const uint32_t ksteps = a.k / C::BK;
  // K part of the current item: steps k0 .. k0 + nk - 1.
  const uint32_t kpp = (ksteps + ksplit - 1) / ksplit;
  uint32_t ctile = 0, kp = 0, k0 = 0, nk = ksteps;
  const uint32_t wm = wave / C::WN, wn = wave % C::WN;

  // Per-lane copy sources of the current tile, loop-invariant within it: a
  // k-step only moves a uniform base, so copies address memory as "scalar
  // base + 32-bit lane offset".  Tile (t, kb) of an operand sits at byte
  // (t * 2 + kb) * 1024 of its half of the stage.  Rows past M and stripes
  // past N repeat the last valid one; their results are never stored.
  uint32_t aoff[C::A_COPIES], boff[C::B_COPIES];
  uint32_t m0 = 0, T0 = 0;
  auto setup = [&](uint32_t id) {
    const uint32_t item = total % 8 == 0 ? (id % 8) * (total / 8) + id / 8 : id;
    const uint32_t tile = item / ksplit;
    ctile = tile;
    kp = item % ksplit;
    k0 = kp * kpp;
    nk = min(ksteps, k0 + kpp) - k0;
    const uint32_t bm = tile % mblocks, bn = tile / mblocks;
    m0 = bm * C::BM;
    T0 = bn * (C::BN / 16);
    // A stage: 128 k-bytes of each of the block's rows, row-major (row r at
    // r * 128), its eight 16-byte chunks XOR-swizzled with (r >> 1) & 7.
    // Each copy moves 8 whole rows: lane L fills slot L % 8 of row L / 8
    // from the row's chunk (L % 8) ^ swizzle, so every 8 lanes read one full
    // 128-byte line of x, and the 16 rows an MFMA operand read touches (at
    // one chunk) land in 16 different bank groups.
#pragma unroll
    for (uint32_t i = 0; i < C::A_COPIES; ++i) {
      const uint32_t r = (i * C::CW + wave % C::CW) * 8 + lane / 8;
      const uint32_t m = min(m0 + r, a.m - 1);
      aoff[i] = m * uint32_t(a.ldxq) + (((lane % 8) ^ ((r >> 1) & 7)) * 16);
    }
#pragma unroll
    for (uint32_t i = 0; i < C::B_COPIES; ++i) {
      const uint32_t c = min(i * C::CW + wave % C::CW, C::B_TILES - 1);
      const uint32_t t = c / 2, kb = c % 2;
      const uint32_t T = min(T0 + t, stripes - 1);
      boff[i] = (T * a.units + kb) * 1024 + lane * 16;
    }
  };
  // LDS: ASTAGES A buffers, then BSTAGES B buffers.
  auto a_buf = [&](uint32_t ks) { return lds + (ks % C::ASTAGES) * C::A_BYTES; };
  auto b_buf = [&](uint32_t ks) {
    return lds + C::ASTAGES * C::A_BYTES + (ks % C::BSTAGES) * C::B_BYTES;
  };
  // Operand buffers (byte extents below 4 GiB: checked by the launcher).
  const __amdgpu_buffer_rsrc_t abuf =
      byte_buffer(a.xq, uint32_t(uint64_t(a.m) * a.ldxq));
  const __amdgpu_buffer_rsrc_t bbuf =
      byte_buffer(a.tiles, uint32_t(uint64_t(stripes) * a.units * 1024));
  // With the ping-pong loop the first CW waves copy A and the last CW B;
  // otherwise every wave copies both.
  const bool a_copier = !C::PP || wave < C::CW;
  const bool b_copier = !C::PP || wave >= C::CW;
  const uint32_t cwave = wave % C::CW;
  // Copies of step ks into the given stage (default: the ring slot of ks).
  auto copy_a_to = [&](uint32_t ks, char *st) {
    if (!a_copier) {
      return;
    }
#pragma unroll
    for (uint32_t i = 0; i < C::A_COPIES; ++i) {
      dma16_buf(abuf, aoff[i], ks * C::BK, st + (i * C::CW + cwave) * 1024);
    }
  };
  auto copy_b_to = [&](uint32_t ks, char *st) {
    if (!b_copier) {
      return;
    }
#pragma unroll
    for (uint32_t i = 0; i < C::B_COPIES; ++i) {
      if (C::B_EVEN || i * C::CW + cwave < C::B_TILES) {
        dma16_buf(bbuf, boff[i], ks * 2048, st + (i * C::CW + cwave) * 1024);
      }
    }
  };
  auto copy_a = [&](uint32_t ks) { copy_a_to(ks, a_buf(ks)); };
  auto copy_b = [&](uint32_t ks) { copy_b_to(ks, b_buf(ks)); };
  constexpr uint32_t BAHEAD = C::BSTAGES - 1;  // k-steps B runs ahead
  constexpr uint32_t AAHEAD = C::ASTAGES - 1;  // k-steps A runs ahead
  // The first copies of the item's K part (absolute steps k0 ..) into the
  // first stages.
  auto prologue = [&]() {
#pragma unroll
    for (uint32_t b = 0; b < AAHEAD; ++b) {
      if (b < nk) {
        copy_a_to(k0 + b, a_buf(b));
      }
    }
#pragma unroll
    for (uint32_t b = 0; b < BAHEAD; ++b) {
      if (b < nk) {
        copy_b_to(k0 + b, b_buf(b));
      }
    }
  };
  const uint32_t swz = (lane % 16) >> 1 & 7;
  const uint32_t a_lo = ((lane / 16) ^ swz) * 16;
  const uint32_t a_hi = ((4 + lane / 16) ^ swz) * 16;
  auto a_operand = [&](const char *rows, uint32_t i) {
    const char *p = rows + i * 16 * 128;
    const u32x4 lo = *reinterpret_cast<const u32x4 *>(p + a_lo);
    const u32x4 hi = *reinterpret_cast<const u32x4 *>(p + a_hi);
    const u32x8 v = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    return __builtin_bit_cast(i32x8, v);
  };

  uint32_t id = blockIdx.x;
  if (id >= total) {
    return;
  }
  setup(id);
  prologue();
  const uint32_t ncol = lane % 16, rq = 4 * (lane / 16);
  float sn[C::TN], sm[C::TM][4];
  // Row and column scales of the current tile's epilogue (lane: rows
  // 4 (lane / 16) + r and column lane % 16 of each 16 x 16 tile).
  auto load_scales = [&]() {
    const uint32_t mw = m0 + wm * C::TM * 16, nw = (T0 + wn * C::TN) * 16;
#pragma unroll
    for (uint32_t j = 0; j < C::TN; ++j) {
      sn[j] = a.scales[min(nw + j * 16 + ncol, stripes * 16 - 1)];
    }
#pragma unroll
    for (uint32_t i = 0; i < C::TM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sm[i][r] = a.xs[min(mw + i * 16 + rq + r, a.m - 1)];
      }
    }
  };
  while (true) {
  if constexpr (C::EARLY_SCALES) {
    load_scales();  // waited for with the first copies, below
  }
  f32x4 acc[C::TM][C::TN];
#pragma unroll
  for (uint32_t i = 0; i < C::TM; ++i) {
#pragma unroll
    for (uint32_t j = 0; j < C::TN; ++j) {
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  gemm_barrier();

  if constexpr (C::PP) {
    static_assert(C::WAVES == 8, "ping-pong: 8 waves");
    // Waves 0-3 (group 0) and 4-7 (group 1) sit one of each per SIMD, and
    // run the same loop -- read a step's operands from LDS, barrier, run
    // its MFMAs, barrier -- with group 1 one phase behind (an extra barrier
    // before its loop, matched by one after group 0's).  While one wave of
    // a SIMD waits on LDS the other keeps the matrix core busy.  Group 0
    // issues the A copies for step ks + AAHEAD (ASTAGES - 1 steps ahead:
    // their stage was last read by group 1 in the phase just ended) before
    // it reads step ks, and waits for step ks + 1's before the barrier that
    // ends its MFMA phase; group 1 issues the B copies for step ks + BAHEAD
    // (two steps ahead with three B stages) before it reads step ks and
    // waits for step ks + 1's before the barrier that ends its read phase.
    // Waits count copies, so the later steps' stay in flight.
    // Each phase then carries about half of a step's copy instructions.
    // The copies slow the loop in proportion to the instructions issued in
    // one phase, not by their latency (waiting for them costs ~1 %): on
    // MI355X at M=2048, N=28672, with group 0 issuing every copy into two B
    // stages, a k-step of every CU's tile took 1.31 us (K sweep 4096 ->
    // 8192) and the launch 207 us; split, 1.14 us and 197 us.
    const bool g1 = wave >= C::WAVES / 2;
    i32x8 af[C::TM], bf[C::TN];
    if (g1) {
      gemm_barrier();
    }
    // The stages being read, kept as counters (A: ks % ASTAGES, B:
    // ks % BSTAGES; an, bn: the stages of steps ks + AAHEAD, ks + BAHEAD).
    uint32_t st = 0, sb = 0, an = AAHEAD, bn = BAHEAD;
    char *const bstages = lds + C::ASTAGES * C::A_BYTES;
#pragma clang loop unroll(disable)
    for (uint32_t ks = 0; ks < nk; ++ks) {
      // Group 0 copies A for step ks + 1 (its stage was last read in the
      // phase just ended), group 1 B for step ks + 2 (its stage held step
      // ks - 1, read by both groups before this phase); ks counts the
      // item's K part, k0 + ks is the absolute step.
      if (!g1 && ks + AAHEAD < nk) {
        copy_a_to(k0 + ks + AAHEAD, lds + an * C::A_BYTES);
      }
      if (g1 && ks + BAHEAD < nk) {
        copy_b_to(k0 + ks + BAHEAD, bstages + bn * C::B_BYTES);
      }
      const char *As = lds + st * C::A_BYTES + (wm * C::TM * 16 + lane % 16) * 128;
      const char *Bs = bstages + sb * C::B_BYTES + (wn * C::TN * 2) * 1024 + lane * 16;
      st = st == C::ASTAGES - 1 ? 0u : st + 1u;
      an = an == C::ASTAGES - 1 ? 0u : an + 1u;
      sb = sb == C::BSTAGES - 1 ? 0u : sb + 1u;
      bn = bn == C::BSTAGES - 1 ? 0u : bn + 1u;
#pragma unroll
      for (uint32_t i = 0; i < C::TM; ++i) {
        af[i] = a_operand(As, i);
      }
#pragma unroll
      for (uint32_t j = 0; j < C::TN; ++j) {
        bf[j] = lds_operand(Bs + j * 2048);
      }
      // Group 1: step ks + 1's B copies have landed before the barrier
      // after which group 0 reads them; those of the later steps stay in
      // flight (near the end of the part, when fewer were issued, wait for
      // all).
      if (g1) {
        if (ks + BAHEAD < nk) {
          wait_vm<(BAHEAD - 1) * C::B_COPIES>();
        } else {
          __builtin_amdgcn_s_waitcnt(0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      gemm_barrier();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (uint32_t i = 0; i < C::TM; ++i) {
#pragma unroll
        for (uint32_t j = 0; j < C::TN; ++j) {
          acc[i][j] = mfma_fp8_k128(af[i], bf[j], acc[i][j]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (!g1) {
        // Step ks + 1's A copies have landed; with more A stages those of
        // the later steps stay in flight.
        if (AAHEAD > 1 && ks + AAHEAD < nk) {
          wait_vm<(AAHEAD - 1) * C::A_COPIES>();
        } else {
          __builtin_amdgcn_s_waitcnt(0);
        }
      }
      gemm_barrier();
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!g1) {
      gemm_barrier();
    }
  } else
  for (uint32_t ks = 0; ks < ksteps; ++ks) {
    // Copies needed by step ks + 1 are issued before those two steps
    // ahead: the in-order vector-memory counter then proves the former
    // (and everything older) landed while the latter stay in flight.
    const bool two_more = ks + 2 < ksteps;
    if (ks + 1 < ksteps) {
      if (AAHEAD == 1) {
        copy_a(ks + 1);
      }
      if (BAHEAD == 1) {
        copy_b(ks + 1);
      }
    }
    if (two_more) {
      if (AAHEAD == 2) {
        copy_a(ks + 2);
      }
      if (BAHEAD == 2) {
        copy_b(ks + 2);
      }
    }
    // Lane l's operand of m-tile i: row 16 i + l % 16 of the wave's rows,
    // k-bytes 16 (l / 16) .. (lo) and 64 + 16 (l / 16) .. (hi).
    const char *As = a_buf(ks) + (wm * C::TM * 16 + lane % 16) * 128;
    const char *Bs = b_buf(ks) + (wn * C::TN * 2) * 1024 + lane * 16;
    i32x8 bf[C::TN];
#pragma unroll
    for (uint32_t j = 0; j < C::TN; ++j) {
      bf[j] = lds_operand(Bs + j * 2048);
    }
    // The A operand of m-tile i + 1 is read while the MFMAs of m-tile i run.
    i32x8 af = a_operand(As, 0);
#pragma unroll
    for (uint32_t i = 0; i < C::TM; ++i) {
      i32x8 an = af;
      if (i + 1 < C::TM) {
        an = a_operand(As, i + 1);
      }
#pragma unroll
      for (uint32_t j = 0; j < C::TN; ++j) {
        acc[i][j] = mfma_fp8_k128(af, bf[j], acc[i][j]);
      }
      af = an;
    }
    // Copies still allowed in flight: those issued for step ks + 2.  When
    // the waves do not split B evenly, the last B round is issued by the
    // first B_TILES % WAVES waves only.
    constexpr uint32_t ahead2 = (AAHEAD == 2 ? C::A_COPIES : 0) +
                                (BAHEAD == 2 ? C::B_COPIES : 0);
    if constexpr (ahead2 > 0) {
      if (!two_more) {
        __builtin_amdgcn_s_waitcnt(0);
      } else if (BAHEAD == 1 || C::B_EVEN || wave < C::B_TILES % C::CW) {
        wait_vm<ahead2>();
      } else {
        wait_vm<ahead2 - 1>();
      }
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    gemm_barrier();
  }

  // The main loop ended on a barrier: every operand stage is free.
  if constexpr (SPLIT) {
    {
      // Split K: every part stores its fp32 sums; the last part of the tile
      // to arrive adds all parts in part order (the result does not depend
      // on the arrival order) and runs the epilogue, the others move on.
      // The parts of a tile may run on different XCDs, whose L2 caches are
      // not coherent: the sums are stored and loaded with the
      // system-coherent policy (sc0 sc1: to and from memory, never a stale
      // L2 line), the stores complete (vmcnt 0) before this workgroup's
      // device-scope counter increment, and the counter elects the one
      // workgroup that saw every other part's increment, so every other
      // part's stores had completed before it loads them.  The finisher
      // resets the counter for the next call.
      const __amdgpu_buffer_rsrc_t pbuf = byte_buffer(a.part, a.part_bytes);
      constexpr uint32_t WB = C::TM * C::TN * kWave * 16;  // bytes per wave and part
      const uint32_t lane_off = wave * WB + lane * 16;
      const uint32_t part0 = ctile * ksplit * (C::WAVES * WB);
#pragma unroll
      for (uint32_t i = 0; i < C::TM; ++i) {
#pragma unroll
        for (uint32_t j = 0; j < C::TN; ++j) {
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4, acc[i][j]), pbuf,
              part0 + kp * (C::WAVES * WB) + lane_off + (i * C::TN + j) * (kWave * 16), 0,
              kScGemm);
        }
      }
      __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores completed
      gemm_barrier();
      // The flag lives in the last B stage, which no copy targets until the next
      // item's prologue (issued below, after the flag is read).
      uint32_t *flag = reinterpret_cast<uint32_t *>(lds + C::ASTAGES * C::A_BYTES +
                                                    (C::BSTAGES - 1) * C::B_BYTES);
      if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(a.cnt + ctile, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev + 1 == ksplit;
        if (last) {
          __hip_atomic_store(a.cnt + ctile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        *flag = last ? 1u : 0u;
      }
      gemm_barrier();
      if (__builtin_amdgcn_readfirstlane(*flag) == 0u) {
        const uint32_t nxt = id + gridDim.x;
        if (nxt >= total) {
          break;
        }
        id = nxt;
        gemm_barrier();  // every wave has read the flag
        setup(id);
        prologue();
        continue;
      }
#pragma unroll
      for (uint32_t i = 0; i < C::TM; ++i) {
#pragma unroll
        for (uint32_t j = 0; j < C::TN; ++j) {
          f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
          for (uint32_t q = 0; q < ksplit; ++q) {
            const f32x4 t =
                q == kp ? acc[i][j]
                        : __builtin_bit_cast(
                              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                         pbuf,
                                         part0 + q * (C::WAVES * WB) + lane_off +
                                             (i * C::TN + j) * (kWave * 16),
                                         0, kScGemm));
            v += t;
          }
          acc[i][j] = v;
        }
      }
    }
  }
  const uint32_t cm0 = m0, cT0 = T0;
  const uint32_t next = id + gridDim.x;
  const bool more = next < total;
  // The epilogue leaves the stages of the next tile's first copies alone
  // (its LDS chunks lie past the stages, or in the last A stage in the
  // ping-pong blocks), so those copies are issued during it: after the scales below
  // are in use (waiting for them then does not wait for the copies) and
  // before the stores.
  auto issue_next = [&]() {
    if (more) {
      setup(next);
      prologue();
    }
  };

  // Epilogue: lane holds rows 4 * (lane / 16) + r, column lane % 16 of each
  // 16 x 16 tile.  Scales are gathered first (independent loads in flight
  // together).
  const uint32_t mw = cm0 + wm * C::TM * 16, nw = (cT0 + wn * C::TN) * 16;
  if constexpr (!C::EARLY_SCALES) {
    load_scales();
  }
  if (!a.y_f32 && a.y_vec) {
    // Per m-tile, each 16 x 16 MFMA result goes to the wave's LDS chunk as
    // bf16: without a fused epilogue, and for silu(gate) * up (the up
    // columns from lane ^ 8), straight from the MFMA layout, one 2-byte
    // write per row; with a residual, through a quad transpose to one row x
    // four columns per lane (fp32), where the residual is read as one
    // 4-column vector, written as 8 bytes.  The chunk's rows then leave as 16-byte
    // segments, each row of the wave's tile one contiguous run, through
    // non-temporal stores (the output is not read again by this launch, and
    // whole segments need no write combining in L2).  Measured on MI355X at
    // M=2048, N=28672, K=4096: 8-byte direct stores 267-272 us, the whole
    // tile staged with plain stores 273-280 us, staged with non-temporal
    // stores 259-261 us, per m-tile chunk with non-temporal stores 245-247.
    constexpr bool gated = EPI == kEpiSiluMul;
    constexpr bool resid = EPI == kEpiResidual;
    uint16_t *chunk = reinterpret_cast<uint16_t *>(lds + C::CHUNK_BASE) +
                      wave * (C::CHUNK_BYTES / 2);
    const uint32_t row = rq + lane % 4, c4 = (ncol / 4) * 4;
    // Gated: lanes with c4 < 8 hold gate columns, those with c4 >= 8 the
    // matching up columns; the output has 8 features per 16-column tile.
    constexpr uint32_t tw = gated ? 8 : 16;  // output columns per tile
    constexpr uint32_t lpr = C::TN * tw / 8, segs = 16 * lpr;
    const uint32_t n0 = gated ? nw / 2 : nw;
    const uint32_t nlim = gated ? a.epi.n_out : a.n;
    // Residual read as 4-element vectors when rows and base allow it.
    const bool res_vec =
        resid && reinterpret_cast<uintptr_t>(a.epi.res) % 16 == 0 && a.epi.ldr % 4 == 0;
#pragma unroll
    for (uint32_t i = 0; i < C::TM; ++i) {
      const uint32_t m = mw + i * 16 + row;
      f32x4 rv[C::TN];
      if constexpr (resid) {
        // All of the m-tile's residual loads are issued before any is used.
#pragma unroll
        for (uint32_t j = 0; j < C::TN; ++j) {
          const uint32_t n = nw + j * 16 + c4;
          rv[j] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (m < a.m) {
            const uint64_t ri = uint64_t(m) * a.epi.ldr + n;
            const float *rf = static_cast<const float *>(a.epi.res) + ri;
            const uint16_t *rh = static_cast<const uint16_t *>(a.epi.res) + ri;
            if (res_vec && n + 4 <= a.n) {
              if (a.epi.res_f32) {
                rv[j] = *reinterpret_cast<const f32x4 *>(rf);
              } else {
                const u32x2 h = *reinterpret_cast<const u32x2 *>(rh);
                rv[j] = f32x4{bits_f32(h.x << 16), bits_f32(h.x & 0xffff0000u),
                              bits_f32(h.y << 16), bits_f32(h.y & 0xffff0000u)};
              }
            } else {
              for (uint32_t e = 0; e < 4 && n + e < a.n; ++e) {
                rv[j][e] = a.epi.res_f32 ? rf[e] : bf16_to_f32(rh[e]);
              }
            }
          }
        }
      }
#pragma unroll
      for (uint32_t j = 0; j < C::TN; ++j) {
        f32x4 v;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r] = a.alpha * ((sm[i][r] * sn[j]) * acc[i][j][r]);
        }
        if constexpr (!resid && !gated) {
          // No fused epilogue: the four rows go to the chunk straight from
          // the MFMA layout (lane: rows rq .. rq + 3 of column ncol), one
          // 2-byte write each, instead of a lane-quad transpose.
          const uint32_t p01 = f32x2_to_bf16x2(v[0], v[1]);
          const uint32_t p23 = f32x2_to_bf16x2(v[2], v[3]);
          uint16_t *c0 = chunk + rq * C::OUT_STRIDE + j * 16 + ncol;
          c0[0] = uint16_t(p01);
          c0[C::OUT_STRIDE] = uint16_t(p01 >> 16);
          c0[2 * C::OUT_STRIDE] = uint16_t(p23);
          c0[3 * C::OUT_STRIDE] = uint16_t(p23 >> 16);
          continue;
        }
        if constexpr (gated) {
          // SiLU-gate in the MFMA layout: lane l (column ncol < 8) holds
          // gate values whose up partners sit in lane l ^ 8 (column
          // ncol + 8, the same rows); its four output rows go to the chunk
          // at feature column 8 j + ncol as 2-byte writes.
          f32x4 h;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float up = dpp_f32<kDppXor8>(v[r]);
            h[r] = silu_f32(v[r]) * up;
          }
          if (ncol < 8) {
            const uint32_t p01 = f32x2_to_bf16x2(h[0], h[1]);
            const uint32_t p23 = f32x2_to_bf16x2(h[2], h[3]);
            uint16_t *c0 = chunk + rq * C::OUT_STRIDE + j * 8 + ncol;
            c0[0] = uint16_t(p01);
            c0[C::OUT_STRIDE] = uint16_t(p01 >> 16);
            c0[2 * C::OUT_STRIDE] = uint16_t(p23);
            c0[3 * C::OUT_STRIDE] = uint16_t(p23 >> 16);
          }
          continue;
        }
        f32x4 t = quad_transpose_f32(v, lane);
        if constexpr (resid) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            t[e] += rv[j][e];
          }
        }
        *reinterpret_cast<u32x2 *>(chunk + row * C::OUT_STRIDE + j * 16 + c4) =
            pack_bf16x4(t);
      }
      if (i == 0) {
        issue_next();
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's chunk is written
#pragma unroll
      for (uint32_t it = 0; it < (segs + kWave - 1) / kWave; ++it) {
        const uint32_t seg = it * kWave + lane;
        if (segs % kWave != 0 && seg >= segs) {
          break;
        }
        const uint32_t rr = seg / lpr, c8 = (seg % lpr) * 8;
        const u32x4 w = *reinterpret_cast<const u32x4 *>(
            chunk + rr * C::OUT_STRIDE + c8);
        const uint32_t mo = mw + i * 16 + rr, n = n0 + c8;
        uint16_t *dst = static_cast<uint16_t *>(a.y) + uint64_t(mo) * a.ldy + n;
        if (mo < a.m) {
          if (n + 8 <= nlim) {
            __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(dst));
          } else {
            const uint32_t e4[4] = {w.x, w.y, w.z, w.w};
            for (uint32_t e = 0; e < 8 && n + e < nlim; ++e) {
              dst[e] = static_cast<uint16_t>(e4[e / 2] >> (16 * (e % 2)));
            }
          }
        }
      }
      // The next m-tile's chunk writes follow these reads in the wave's
      // in-order LDS queue.
    }
  } else {
    issue_next();
#pragma unroll
    for (uint32_t i = 0; i < C::TM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t m = mw + i * 16 + rq + r;
#pragma unroll
        for (uint32_t j = 0; j < C::TN; ++j) {
          const uint32_t n = nw + j * 16 + ncol;
          const float v = a.alpha * ((sm[i][r] * sn[j]) * acc[i][j][r]);
          store_out<EPI>(a.y, a.ldy, a.y_f32, a.epi, a.n, m, n, v, m < a.m);
        }
      }
    }
  }
  if (!more) {
    break;
  }
  id = next;
  }  // tiles
}

// 256 x 256: 2 waves of 128 rows x 4 of 64 columns, ping-pong with three B
// stages (LDS 160 KiB; the epilogue chunks fit A stage 1 at 64 columns per
// wave).  Measured on MI355X against the same block without the ping-pong
// loop: M=2048 N=8192 54.5 against 57.5 us, M=4096 N=4096 53.1 against 56.8
// us, M=2048 N=16384 110 against 116.4 us.
using GemmLarge = GemmCfg<256, 256, 2, 4, 3, 2, true>;
// 224 columns: 4 waves of 64 rows x 2 of 112 columns, ping-pong main loop.
// For N = 28672 (and any N with whole 224-column blocks) the tile count
// becomes a multiple of the CU count where 256-column tiles leave the last
// round half empty.  Measured on MI355X at M=2048, N=28672: ping-pong
// 215-220 against 232-235 us (per 128-deep k-step of every CU's tile 1.32
// against 1.48-1.54 us, from a K sweep).  Three B stages with the copy
// issue split between the groups: 196-197 against 207 us, 1.14
// against 1.31 us per k-step; a third B stage with group 0 still issuing
// every copy gained nothing.
using GemmNarrow = GemmCfg<256, 224, 4, 2, 3, 2, true>;
// 192 columns: 4 waves of 64 rows x 2 of 96 columns, ping-pong, for grids
// where it fills the last round (M = 2048, N = 6144: 256 tiles, one full
// round; 48.5 against 54.1 us without the ping-pong loop).
using GemmNarrow192 = GemmCfg<256, 192, 4, 2, 3, 2, true>;
// 8 waves of 64 x 32; 2 workgroups per CU.  The ping-pong loop measured
// level or slower here (two workgroups already interleave on each SIMD)
// and needs more than the 128 registers per wave two workgroups allow.
using GemmMid = GemmCfg<128, 128, 2, 4>;
// 128 columns: 4 waves of 64 rows x 2 of 64 columns, ping-pong with three B
// and three A stages (144 KiB), one workgroup per CU, for N = 4096-class
// grids (one full round of 256 x 128 tiles at M = 2048).
using GemmNarrow128 = GemmCfg<256, 128, 4, 2, 3, 3, true>;
// 64 columns: 4 waves of 64 rows x 2 of 32 columns, for the smallest grids;
// three B and three A stages (120 KiB).  With A copied two k-steps ahead
// instead of one (both widths; MI355X, K = 4096 unless noted): M=120
// N=14336 24.0 against 26.9 us, M=768 N=4096 23.3 against 25.5, M=256
// N=14336 27.1 against 29.9, M=512 N=4096 K=14336 48.2 against 51.5, M=256
// N=4096 18.7 against 19.5; M=2048 N=4096 level.
using GemmNarrow64 = GemmCfg<256, 64, 4, 2, 3, 3, true>;
// 128 and 64 rows by 64 or 128 columns for short prompts (block_m_for):
// ping-pong, three A and three B stages; waves of 32 x 32 (128 x 64, 4 x 2
// waves), 32 x 16 (64 x 64, 2 x 4), 64 x 32 (128 x 128, 2 x 4) and 32 x 32
// (64 x 128, 2 x 4; its epilogue chunks lie past the stages).
using GemmSmall128 = GemmCfg<128, 64, 4, 2, 3, 3, true>;
using GemmSmall64 = GemmCfg<64, 64, 2, 4, 3, 3, true>;
using GemmSmall128W = GemmCfg<128, 128, 2, 4, 3, 3, true>;
using GemmSmall64W = GemmCfg<64, 128, 2, 4, 3, 3, true>;


// Block width (256, 224 or 192 columns, 256 rows) whose rounds of
// one-workgroup-per-CU tiles finish first: the kernel takes ceil(tiles /
// CUs) rounds, each as long as one tile, and a tile's time scales with its
// width, so cost = rounds x width, ties to the wider block.
uint32_t gemm_block_n(uint32_t m, uint32_t n, uint32_t cus) {
  const uint64_t mb = (m + 255) / 256;
  uint32_t best = 256;
  uint64_t best_cost = ~uint64_t(0);
  for (uint32_t bn : {256u, 224u, 192u}) {
    const uint64_t tiles = mb * ((n + bn - 1) / bn);
    const uint64_t cost = (tiles + cus - 1) / cus * bn;
    if (cost < best_cost) {
      best_cost = cost;
      best = bn;
    }
  }
  return best;
}

// 128 x 128 blocks, two workgroups per CU, when the large blocks would
// leave CUs idle: a round of them (two tiles per CU) takes ~0.8 of a round
// of large blocks (their per-CU rate is ~0.7-0.75 of the large blocks',
// from twice the operand traffic per flop), so they win whenever they need
// fewer rounds.  Measured on MI355X, K = 4096 unless noted: M=2048 N=4096
// 52 -> 37 us, N=4096 K=14336 139 -> 114 us, M=1024 N=4096 46 -> 30 us;
// N=6144 (one round of large blocks, two of mid) stays with the large
// blocks, 52-54 against 61 us.
bool gemm_use_mid(uint32_t m, uint32_t n, uint32_t cus) {
  const uint64_t mb = (m + 255) / 256;
  uint64_t rounds_large = ~uint64_t(0);
  for (uint32_t bn : {256u, 224u, 192u}) {
    const uint64_t tiles = mb * ((n + bn - 1) / bn);
    rounds_large = std::min(rounds_large, (tiles + cus - 1) / cus);
  }
  const uint64_t tmid = uint64_t((m + 127) / 128) * ((n + 127) / 128);
  const uint64_t rounds_mid = (tmid + 2 * cus - 1) / (2 * cus);
  return double(rounds_mid) * 0.82 < double(rounds_large) * 0.95;
}

// Where the 128 x 128 blocks would win over the wide ones, 256 x 128 ping-pong
// blocks (one workgroup per CU) win over them in turn whenever their grid
// needs no more rounds: one 256 x 128 tile takes less time than a round of
// two 128 x 128 tiles per CU, even with most CUs idle.  Measured on MI355X at
// K = 4096 (against 128 x 128): M=2048 N=4096 33.1 against 38.2 us (K=14336:
// 100.6 against 120.5 us), M=1024 27.5 against 30.5, M=256 26.8 against 29.6
// (16 tiles), M=512 N=6144 27.7 against 30.7, M=256 N=28672 43.3 against
// 48.6 us.
bool gemm_use_128(uint32_t m, uint32_t n, uint32_t cus) {
  const uint64_t t128 = uint64_t((m + 255) / 256) * ((n + 127) / 128);
  const uint64_t tmid = uint64_t((m + 127) / 128) * ((n + 127) / 128);
  const uint64_t r128 = (t128 + cus - 1) / cus;
  const uint64_t rmid = (tmid + 2 * cus - 1) / (2 * cus);
  return r128 <= rmid;
}

// Among those, 256 x 64 blocks when their grid needs no more rounds than the
// 256 x 128 one: on grids this small a tile's time is set by its k-loop, not
// by its width.  Measured on MI355X at K = 4096 (against 256 x 128): M=256
// N=4096 23.0 against 27.0 us, M=512 N=4096 23.6 against 27.0, M=256
// N=6144 23.9 against 27.3, M=768 N=4096 25.2 against 27.4, M=1024 N=4096
// 26.8 against 27.7 (K=14336: 83.0 against 85.2), M=256 N=14336 29.7
// against 30.0.
bool gemm_use_64(uint32_t m, uint32_t n, uint32_t cus) {
  const uint64_t mb = (m + 255) / 256;
  const uint64_t r64 = (mb * ((n + 63) / 64) + cus - 1) / cus;
  const uint64_t r128 = (mb * ((n + 127) / 128) + cus - 1) / cus;
  return r64 <= r128;
}

// Split K over workgroups on grids of few tiles (ping-pong blocks, one round,
// at most half of the CUs busy): a tile's k-loop then runs at the copy rate
// of one CU however many CUs idle, so the idle CUs take parts of K, at
// least 16 steps each, and the last part of a tile to finish adds the parts.
// K parts for `tiles` one-workgroup tiles of bm x bn (1: no split).
// ULLM_GEMM_SPLIT=0 (read only by a -DULLM_TUNING build) turns it off.
uint32_t split_parts(uint32_t tiles, uint32_t k, uint32_t cus, uint32_t bm,
                     uint32_t bn) {
  const char *env = tuning_env("ULLM_GEMM_SPLIT");
  if (env != nullptr && env[0] == '0') {
    return 1;
  }
  // A part of fewer than 16 k-steps does not pay for its partial-sum round
  // trip (store, counter, reload by the finisher): with 8 the measured
  // M=300 N=2000 K=2048 launch took 14.3 us split against 14.0 unsplit.
  // The 64 x 64 blocks' partial sums are small enough for parts of 8
  // (M=64 N=4096 K=4096 11.2 against 12.0 us, M=16 10.9 against 11.8).
  uint32_t min_steps = bm * bn <= 64 * 64 ? 8 : 16;
  if (const char *v = tuning_env("ULLM_GEMM_SPLIT_STEPS")) {
    min_steps = std::max(1, std::atoi(v));
  }
  const uint32_t ksteps = k / 128;
  if (ksteps < 2 * min_steps || 2 * tiles > cus || tiles * 4 > kGemmCounterBytes) {
    return 1;
  }
  uint32_t ks = std::min(cus / tiles, ksteps / min_steps);
  // Every part holds at least one step.
  while (ks > 1 && (ks - 1) * ((ksteps + ks - 1) / ks) >= ksteps) {
    --ks;
  }
  const uint64_t part = uint64_t(tiles) * ks * bm * bn * 4;
  return ks < 2 || part >= (uint64_t(1) << 31) ? 1 : ks;
}

void plan_split(GemmPlan &p, uint32_t k, uint32_t cus) {
  p.ksplit = 1;
  if (p.grid < p.tiles) {
    return;  // persistent: every CU already busy
  }
  const uint32_t ks = split_parts(p.tiles, k, cus, p.block_m, p.block_n);
  if (ks > 1) {
    p.ksplit = ks;
    p.grid = p.tiles * ks;
  }
}

// Rows of the 64- or 128-column blocks (256, 128 or 64).  On the grids these blocks
// serve (one round or a few) a workgroup's k-loop runs at the rate one CU
// copies its operands into LDS, ~60 GB/s per CU whatever the block's MFMA
// work: a k-step of a 256 x 64 block (40 KiB) took ~0.67 us, of a 128 x 64
// block (24 KiB) ~0.41 us, of a 64 x 64 block (16 KiB) ~0.27 us (MI355X,
// every CU busy).  So the launch takes about rounds x k-steps per
// workgroup x bytes per k-step, with rows past M costing nothing (they
// repeat the last row, an L2 hit), plus, with K split, the partial sums'
// round trips (in proportion to the block's rows and the parts beyond the
// first: 256-row blocks split 7 ways measured 33.0 against 23.4 us for
// 128-row ones split 4 ways at M=256 N=2048 K=14336); the fewest rows win ties
// (less MFMA work, fewer padded rows).  The 128- and 64-row blocks are
// taken on one round only: over several rounds they lost every time.
// Measured (K = 4096 unless noted; 256 / 128 / 64 rows): M=64 N=4096 18.0 /
// 13.9 / 12.5 us, M=256 N=4096 18.7 / 14.6 / 16.8, M=256 N=6144 20.0 / 18.5
// / 20.5, M=120 N=14336 23.9 / 20.4 / 22.8, M=256 N=2048 K=14208 33.0 /
// 23.4 / -, M=256 N=14336 26.7 / 28.9 / 39.9, M=512 N=4096 K=14336 47.5 /
// 55.5 / 64.0, M=768 N=4096 23.3 / 24.6 / 32.6, M=300 N=6000 22.7 / 25.1 /
// 24.3: the model picks the fastest of each.
uint32_t block_m_for(uint32_t bn, uint32_t m, uint32_t n, uint32_t k, uint32_t cus) {
  if (const char *v = tuning_env("ULLM_GEMM_BM")) {
    const int bm = std::atoi(v);
    if (bm == 64 || bm == 128 || bm == 256) {
      return uint32_t(bm);
    }
  }
  const uint64_t ksteps = k / 128;
  uint32_t best = 256;
  uint64_t best_cost = ~uint64_t(0);
  for (uint32_t bm : {64u, 128u, 256u}) {
    const uint32_t tiles = ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    if (bm < 256 && tiles > cus) {
      continue;
    }
    const uint32_t ks = split_parts(tiles, k, cus, bm, bn);
    const uint64_t rounds = (uint64_t(tiles) * ks + cus - 1) / cus;
    const uint64_t steps = (ksteps + ks - 1) / ks;
    const uint64_t cost = rounds * steps * (std::min(bm, m) + bn) + 5 * bm * (ks - 1);
    if (cost < best_cost) {
      best_cost = cost;
      best = bm;
    }
  }
  return best;
}

template <class C>
void fill_plan(GemmPlan &p, uint32_t m, uint32_t n, uint32_t cus,
               bool persist) {
  p.block_m = C::BM;
  p.block_n = C::BN;
  p.tiles = ((m + C::BM - 1) / C::BM) * ((n + C::BN - 1) / C::BN);
  // One workgroup per CU (two for blocks whose LDS fits twice), looping
  // over tiles.
  uint32_t slots = cus * (C::LDS <= 80 * 1024 ? 2 : 1);
  // Tuning override (read only by a -DULLM_TUNING build): ULLM_GEMM_GRID
  // caps the persistent grid.
  if (const char *g = tuning_env("ULLM_GEMM_GRID")) {
    const int v = std::atoi(g);
    if (v > 0 && uint32_t(v) < slots) {
      slots = uint32_t(v);
    }
  }
  p.grid = persist && p.tiles > slots ? slots : p.tiles;
}

// Dynamic-LDS limit of a kernel raised once per (kernel, device).
hipError_t raise_lds_limit(const void *kernel, uint32_t bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void *, int>> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    return e;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({kernel, dev}) != 0) {
    return hipSuccess;
  }
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          int(bytes));
  if (e == hipSuccess) {
    done.insert({kernel, dev});
  }
  return e;
}

template <class C, uint32_t EPI>
hipError_t launch_gemm_lds(const GemmArgs &a, const GemmPlan &p,
                           hipStream_t s) {
  if constexpr (C::PP) {
    if (p.ksplit > 1) {
      const void *ks = reinterpret_cast<const void *>(fp8_gemm_lds_kernel<C, EPI, true>);
      const hipError_t attr = raise_lds_limit(ks, C::LDS);
      if (attr != hipSuccess) {
        return attr;
      }
      hipLaunchKernelGGL((fp8_gemm_lds_kernel<C, EPI, true>), dim3(p.grid),
                         dim3(C::WAVES * kWave), C::LDS, s, a);
      return hipGetLastError();
    }
  }
  const void *k = reinterpret_cast<const void *>(fp8_gemm_lds_kernel<C, EPI, false>);
  const hipError_t attr = raise_lds_limit(k, C::LDS);
  if (attr != hipSuccess) {
    return attr;
  }
  hipLaunchKernelGGL((fp8_gemm_lds_kernel<C, EPI, false>), dim3(p.grid),
                     dim3(C::WAVES * kWave), C::LDS, s, a);
  return hipGetLastError();
}

template <uint32_t EPI>
hipError_t gemm_e(const GemmArgs &a, const GemmPlan &p, bool vec,
                  hipStream_t s) {
  switch (p.kind) {
    case kGemmMid: return launch_gemm_lds<GemmMid, EPI>(a, p, s);
    case kGemmNarrow: return launch_gemm_lds<GemmNarrow, EPI>(a, p, s);
    case kGemmNarrow192: return launch_gemm_lds<GemmNarrow192, EPI>(a, p, s);
    case kGemmNarrow128: return launch_gemm_lds<GemmNarrow128, EPI>(a, p, s);
    case kGemmNarrow64: return launch_gemm_lds<GemmNarrow64, EPI>(a, p, s);
    case kGemmSmall128: return launch_gemm_lds<GemmSmall128, EPI>(a, p, s);
    case kGemmSmall64: return launch_gemm_lds<GemmSmall64, EPI>(a, p, s);
    case kGemmSmall128W: return launch_gemm_lds<GemmSmall128W, EPI>(a, p, s);
    case kGemmSmall64W: return launch_gemm_lds<GemmSmall64W, EPI>(a, p, s);
    case kGemmLarge: return launch_gemm_lds<GemmLarge, EPI>(a, p, s);
    default: break;
  }
  const dim3 grid((a.n + 63) / 64, (a.m + 63) / 64);
  hipLaunchKernelGGL(fp8_gemm_direct_kernel<EPI>, grid, dim3(256), 0, s, a, vec);
  return hipGetLastError();
}

}  // namespace

// The LDS kernel serves every M (rows past M are clamped on load and masked
// on store): at K = 4096 it is 24 us against the direct kernel's 39 us for
// M = 32..96, N = 4096, and 30 against 55-60 us at N = 28672.  The direct
// kernel takes unaligned activations, K not a multiple of 128, and offsets
// past 32 bits.
GemmPlan plan_fp8_gemm(uint32_t m, uint32_t n, uint32_t k, bool vec,
                       bool offsets_fit, uint32_t cus) {
  GemmPlan p{};
  p.ksplit = 1;
  if (!(vec && offsets_fit && k % 128 == 0)) {
    p.kind = kGemmDirect;
    p.block_m = 64;
    p.block_n = 64;
    p.tiles = ((m + 63) / 64) * ((n + 63) / 64);
    p.grid = p.tiles;
    return p;
  }
  // Tuning overrides (read only by a -DULLM_TUNING build): ULLM_GEMM_CFG=mid,
  // ULLM_GEMM_BN=256/224/192/128/64, ULLM_GEMM_BM=256/128/64 (rows of the 64-
  // and 128-column blocks), ULLM_GEMM_PERSIST=0 (one workgroup per tile),
  // ULLM_GEMM_SPLIT=0 and ULLM_GEMM_SPLIT_STEPS (the K split).
  const char *cfg = tuning_env("ULLM_GEMM_CFG");
  const char *bn_env = tuning_env("ULLM_GEMM_BN");
  const char *persist_env = tuning_env("ULLM_GEMM_PERSIST");
  const bool persist = persist_env == nullptr || persist_env[0] != '0';
  const int forced_bn = bn_env ? std::atoi(bn_env) : 0;
  const bool narrow = forced_bn == 0 && cfg == nullptr && gemm_use_mid(m, n, cus) &&
                      gemm_use_128(m, n, cus);
  if (forced_bn == 64 || (narrow && gemm_use_64(m, n, cus))) {
    switch (block_m_for(64, m, n, k, cus)) {
      case 64: p.kind = kGemmSmall64; fill_plan<GemmSmall64>(p, m, n, cus, persist); break;
      case 128: p.kind = kGemmSmall128; fill_plan<GemmSmall128>(p, m, n, cus, persist); break;
      default: p.kind = kGemmNarrow64; fill_plan<GemmNarrow64>(p, m, n, cus, persist); break;
    }
    plan_split(p, k, cus);
    return p;
  }
  if (forced_bn == 128 || narrow) {
    switch (block_m_for(128, m, n, k, cus)) {
      case 64: p.kind = kGemmSmall64W; fill_plan<GemmSmall64W>(p, m, n, cus, persist); break;
      case 128: p.kind = kGemmSmall128W; fill_plan<GemmSmall128W>(p, m, n, cus, persist); break;
      default: p.kind = kGemmNarrow128; fill_plan<GemmNarrow128>(p, m, n, cus, persist); break;
    }
    plan_split(p, k, cus);
    return p;
  }
  if ((cfg != nullptr && cfg[0] == 'm') ||
      (forced_bn == 0 && gemm_use_mid(m, n, cus))) {
    p.kind = kGemmMid;
    fill_plan<GemmMid>(p, m, n, cus, persist);
    return p;
  }
  const uint32_t bn = (forced_bn == 256 || forced_bn == 224 || forced_bn == 192)
                          ? uint32_t(forced_bn)
                          : gemm_block_n(m, n, cus);
  switch (bn) {
    case 224: p.kind = kGemmNarrow; fill_plan<GemmNarrow>(p, m, n, cus, persist); break;
    case 192: p.kind = kGemmNarrow192; fill_plan<GemmNarrow192>(p, m, n, cus, persist); break;
    default: p.kind = kGemmLarge; fill_plan<GemmLarge>(p, m, n, cus, persist); break;
  }
  plan_split(p, k, cus);
  return p;
}

GemmPlan plan_fp8_gemm_call(const void *xq, uint64_t ldxq,
                            const ullm_linear_weight_t *w, uint32_t m) {
  const bool vec = reinterpret_cast<uintptr_t>(xq) % 16 == 0 && ldxq % 16 == 0;
  const bool offsets_fit = uint64_t(m) * ldxq < (uint64_t(1) << 32) &&
                           w->fp8.bytes() < (uint64_t(1) << 32);
  return plan_fp8_gemm(m, static_cast<uint32_t>(w->n), static_cast<uint32_t>(w->k),
                       vec, offsets_fit, device_cu_count());
}

uint64_t gemm_split_bytes(const GemmPlan &p) {
  return p.ksplit > 1
             ? kGemmCounterBytes + uint64_t(p.tiles) * p.ksplit * p.block_m * p.block_n * 4
             : 0;
}

// `p` is plan_fp8_gemm_call for the same xq, ldxq, w and m; with a split,
// `cnt` points at kGemmCounterBytes of counters (zero) and `part` at
// gemm_split_bytes(p) - kGemmCounterBytes bytes for the partial sums.
hipError_t launch_fp8_gemm(const uint8_t *xq, const float *xs, uint64_t ldxq,
                           const ullm_linear_weight_t *w, uint32_t m, void *y,
                           uint64_t ldy, bool y_f32, float alpha,
                           const Epilogue &epi, const GemmPlan &p, uint32_t *cnt,
                           float *part, hipStream_t s) {
  GemmArgs a{};
  a.xq = xq;
  a.xs = xs;
  a.tiles = static_cast<const uint8_t *>(w->tiles);
  a.scales = static_cast<const float *>(w->aux);
  a.y = y;
  a.ldxq = ldxq;
  a.ldy = ldy;
  a.m = m;
  a.n = static_cast<uint32_t>(w->n);
  a.k = static_cast<uint32_t>(w->k);
  a.units = static_cast<uint32_t>(w->fp8.blocks_per_stripe());
  a.alpha = alpha;
  a.y_f32 = y_f32;
  a.y_vec = reinterpret_cast<uintptr_t>(y) % 16 == 0 && ldy % 8 == 0;
  a.epi = epi;
  a.ksplit = p.ksplit;
  if (p.ksplit > 1) {
    if (cnt == nullptr || part == nullptr) {
      return hipErrorInvalidValue;
    }
    a.cnt = cnt;
    a.part = part;
    a.part_bytes = static_cast<uint32_t>(gemm_split_bytes(p) - kGemmCounterBytes);
  }
  const bool vec = reinterpret_cast<uintptr_t>(xq) % 16 == 0 && ldxq % 16 == 0;
  switch (epi.kind) {
    case kEpiSiluMul: return gemm_e<kEpiSiluMul>(a, p, vec, s);
    case kEpiResidual: return gemm_e<kEpiResidual>(a, p, vec, s);
    default: return gemm_e<kEpiNone>(a, p, vec, s);
  }
}

}  // namespace ullm
