// gemv.hip -- decode-shape (M <= 32 per pass) quantized GEMV on gfx950.
//
// Y[m, n] = alpha * sum_k dequant(W)[n, k] * x[m, k], bf16 activations,
// fp32 accumulation, for FP8-E4M3 per-row-scaled and AQ4 g128 weights.
//
// The op is HBM-bound (intensity <= 64 flop/byte at M = 32 against a ridge of
// several hundred), so the kernel is built around streaming the weight tiles
// at full bandwidth and spending as few instructions as possible per byte:
//   * each weight load is one 1 KiB wave-tile (16 bytes per lane, see
//     layout.hpp), already in the lane order the matrix core consumes;
//   * the bytes are unpacked in registers straight into bf16 MFMA operands
//     (FP8 through the hardware scaled convert, AQ4 by OR-ing nibbles into the
//     mantissa of bf16 128.0) and contracted with v_mfma_f32_16x16x32_bf16
//     against bf16 activations read from L2 (x is tiny and shared by every
//     workgroup), so the ALU cost per weight byte is independent of M;
//   * one workgroup owns a 16-row stripe and one 32-row activation block; its
//     waves split K, each streaming a contiguous run of tiles with a batch of
//     loads in flight, and the partial sums meet in LDS once at the end.
// AQ4 uses the identity sum_k (q - z) s x = s * (sum_k (128 + q) x - (128 + z)
// sum_k x) per group: the integer codes stay exact in bf16, the group sum of x
// comes from a second MFMA against a ones operand, and the per-group scale and
// zero are applied once per 128 k in fp32.
#include <cstdlib>
#include <mutex>
#include <algorithm>
#include <unordered_map>

#include "device_common.hpp"
#include "kernels.hpp"

namespace ullm {
namespace {

// Activation row reader.  VEC: rows are 16-byte aligned and K covers every
// unit, so each read is one unconditional 16-byte buffer load.  The buffer
// descriptor spans this workgroup's 32-row activation block; lanes whose row
// is past M get an offset beyond the descriptor's range, which the hardware
// answers with zeros without touching memory -- no branch (a branch around a
// load forces the wait counter to drain) and no wasted traffic at small M.
// The scalar variant handles unaligned views and ragged K.
template <bool VEC>
struct XRow {
  const uint16_t *row;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off;  // byte offset of this lane's row (VEC), out of range if m >= M
  bool valid;
  uint32_t K;
  XRow() = default;
  __device__ __forceinline__ XRow(const uint16_t *x, uint64_t ldx, uint32_t m,
                                  uint32_t M, uint32_t k)
      : row(x + uint64_t(m < M ? m : 0) * ldx), valid(m < M), K(k) {
    if constexpr (VEC) {
      const uint32_t m0 = blockIdx.y * 32;
      const uint32_t rows = min(M - m0, 32u);
      const uint64_t extent = (uint64_t(rows - 1) * ldx + k) * 2;
      rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t *>(x + uint64_t(m0) * ldx), 0,
          static_cast<int>(extent), 0x00020000);
      off = valid ? uint32_t((m - m0) * ldx * 2) : 0x80000000u;
    }
  }
  __device__ __forceinline__ bf16x8 load8(uint32_t k0) const {
    u32x4 r;
    if constexpr (VEC) {
      r = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + k0 * 2, 0, 0));
    } else {
      uint32_t h[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        h[i] = (valid && k0 + i < K) ? row[k0 + i] : 0u;
      }
      r = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                h[6] | (h[7] << 16)};
    }
    return __builtin_bit_cast(bf16x8, r);
  }
};

template <int MT, int WAVES, int EPI = kEpiNone>
__device__ __forceinline__ void reduce_and_store(const GemvArgs &a,
                                                 f32x4 (&acc)[MT], float *red,
                                                 float scale) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      red[((wave * MT + mt) * 4 + r) * kWave + lane] = acc[mt][r];
    }
  }
  __syncthreads();
  const uint32_t T = blockIdx.x;
  const uint32_t m_base = blockIdx.y * 32;
  for (int o = threadIdx.x; o < MT * 256; o += WAVES * kWave) {
    const int mt = o / 256;
    const int mrow = (o % 256) / 16;
    const int ncol = o % 16;
    const int src_lane = ncol + 16 * (mrow / 4);
    const int r = mrow % 4;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      v += red[((w * MT + mt) * 4 + r) * kWave + src_lane];
    }
    const uint32_t m = m_base + mt * 16 + mrow;
    const uint32_t n = T * 16 + ncol;
    store_out<EPI>(a.y, a.ldy, a.y_f32, a.epi, a.n, m, n, a.alpha * (scale * v),
              m < a.m);
  }
}

// Tiles per batch: all activation reads of a batch are issued first, then all
// weight-tile loads, so the consumer waits on an in-order counter that lets the
// remaining tile loads stay in flight.
template <int MT>
constexpr int fp8_batch() { return MT == 1 ? 8 : 4; }
template <int MT>
constexpr int aq4_batch() { return MT == 1 ? 4 : 2; }

template <int MT, int WAVES, bool VEC, int EPI>
__global__ __launch_bounds__(WAVES *kWave) void fp8_gemv_kernel(GemvArgs a) {
  constexpr int B = fp8_batch<MT>();
  __shared__ float red[WAVES * MT * 4 * kWave];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const uint32_t T = blockIdx.x;
  const float rscale =
      static_cast<const float *>(a.aux)[T * 16 + threadIdx.x % 16];
  const uint32_t units = a.units;
  const uint32_t ub = uint32_t(uint64_t(units) * wave / WAVES);
  const uint32_t ue = uint32_t(uint64_t(units) * (wave + 1) / WAVES);
  const uint8_t *stripe = static_cast<const uint8_t *>(a.tiles) +
                          uint64_t(T) * units * 1024 + lane * 16;
  XRow<VEC> xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    xr[mt] = XRow<VEC>(a.x, a.ldx, blockIdx.y * 32 + mt * 16 + lane % 16, a.m,
                       a.k);
  }
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t kl = 16 * (lane / 16);

  auto consume = [&](u32x4 wv, const bf16x8 (&xa)[MT][2]) {
    const u32x2 b01 = e4m3x4_to_bf16x4(wv.x);
    const u32x2 b23 = e4m3x4_to_bf16x4(wv.y);
    const u32x2 b45 = e4m3x4_to_bf16x4(wv.z);
    const u32x2 b67 = e4m3x4_to_bf16x4(wv.w);
    const bf16x8 b0 = __builtin_bit_cast(bf16x8, u32x4{b01.x, b01.y, b23.x, b23.y});
    const bf16x8 b1 = __builtin_bit_cast(bf16x8, u32x4{b45.x, b45.y, b67.x, b67.y});
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[mt] = mfma_bf16(xa[mt][0], b0, acc[mt]);
      acc[mt] = mfma_bf16(xa[mt][1], b1, acc[mt]);
    }
  };
  auto load_x = [&](uint32_t u, bf16x8 (&xa)[MT][2]) {
    const uint32_t k0 = u * 64 + kl;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      xa[mt][0] = xr[mt].load8(k0);
      xa[mt][1] = xr[mt].load8(k0 + 8);
    }
  };

  uint32_t u = ub;
  for (; u + B <= ue; u += B) {
    bf16x8 xa[B][MT][2];
    u32x4 wv[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {
      load_x(u + i, xa[i]);
    }
#pragma unroll
    for (int i = 0; i < B; ++i) {
      wv[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4 *>(stripe + uint64_t(u + i) * 1024));
    }
    // Keep the whole batch of loads ahead of the first use: without this
    // fence the scheduler interleaves loads with their consumers and leaves
    // only one or two tiles in flight.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < B; ++i) {
      consume(wv[i], xa[i]);
    }
  }
  for (; u < ue; ++u) {
    bf16x8 xa[MT][2];
    load_x(u, xa);
    consume(__builtin_nontemporal_load(
                reinterpret_cast<const u32x4 *>(stripe + uint64_t(u) * 1024)),
            xa);
  }
  reduce_and_store<MT, WAVES, EPI>(a, acc, red, rscale);
}

template <int MT, int WAVES, bool VEC, int EPI>
__global__ __launch_bounds__(WAVES *kWave) void aq4_gemv_kernel(GemvArgs a) {
  constexpr int B = aq4_batch<MT>();
  __shared__ float red[WAVES * MT * 4 * kWave];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const uint32_t T = blockIdx.x;
  const uint32_t groups = a.units;
  const uint32_t ub = uint32_t(uint64_t(groups) * wave / WAVES);
  const uint32_t ue = uint32_t(uint64_t(groups) * (wave + 1) / WAVES);
  const uint32_t *stripe = static_cast<const uint32_t *>(a.tiles) +
                           uint64_t(T) * groups * 256 + lane * 4;
  const uint32_t *szs = static_cast<const uint32_t *>(a.aux) +
                        uint64_t(T) * groups * 16 + lane % 16;
  XRow<VEC> xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    xr[mt] = XRow<VEC>(a.x, a.ldx, blockIdx.y * 32 + mt * 16 + lane % 16, a.m,
                       a.k);
  }
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t kl = 8 * (lane / 16);
  const bf16x8 ones = __builtin_bit_cast(
      bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});

  auto consume = [&](u32x4 wv, uint32_t szv, const bf16x8 (&xa)[MT][4]) {
    const bf16x8 b[4] = {nib8_to_bf16_off128(wv.x), nib8_to_bf16_off128(wv.y),
                         nib8_to_bf16_off128(wv.z), nib8_to_bf16_off128(wv.w)};
    const float sf = f16_to_f32(uint16_t(szv & 0xffffu));
    const float zoff = 128.0f + f16_to_f32(uint16_t(szv >> 16));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 p = {0.f, 0.f, 0.f, 0.f};
      f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p = mfma_bf16(xa[mt][j], b[j], p);
        xs = mfma_bf16(xa[mt][j], ones, xs);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[mt][r] += sf * (p[r] - zoff * xs[r]);
      }
    }
  };
  auto load_x = [&](uint32_t g, bf16x8 (&xa)[MT][4]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xa[mt][j] = xr[mt].load8(g * 128 + 32 * j + kl);
      }
    }
  };

  uint32_t g = ub;
  for (; g + B <= ue; g += B) {
    bf16x8 xa[B][MT][4];
    u32x4 wv[B];
    uint32_t szv[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {
      load_x(g + i, xa[i]);
    }
#pragma unroll
    for (int i = 0; i < B; ++i) {
      szv[i] = szs[uint64_t(g + i) * 16];
      wv[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4 *>(stripe + uint64_t(g + i) * 256));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < B; ++i) {
      consume(wv[i], szv[i], xa[i]);
    }
  }
  for (; g < ue; ++g) {
    bf16x8 xa[MT][4];
    load_x(g, xa);
    const uint32_t szv = szs[uint64_t(g) * 16];
    consume(__builtin_nontemporal_load(
                reinterpret_cast<const u32x4 *>(stripe + uint64_t(g) * 256)),
            szv, xa);
  }
  reduce_and_store<MT, WAVES, EPI>(a, acc, red, 1.0f);
}

// ---------------------------------------------------------------------------
// LDS-staged variant.  When the workgroup's activation block (rows x K bf16)
// fits in 64 KiB, it is copied once into LDS with direct global->LDS loads
// (no registers) issued ahead of the first weight batch, and every MFMA A
// operand is read from LDS.  Waves then hold only weight tiles in registers:
// a batch is consumed while the next batch is already in flight.  Rows are
// stored as 16-byte chunks, chunk c of row r at slot c ^ (r & 7), which
// spreads the 16 rows an A read touches over different banks.
// Activation blocks up to this size are staged in LDS (gfx950 has 160 KiB per
// CU; above 64 KiB a kernel needs the dynamic-LDS attribute raised).  Measured
// on MI355X: FP8 gains from staging up to M = 16 at K = 4096 (qkv M=8: 3.1
// against 2.7 TB/s), while AQ4 above 64 KiB loses more to the lower occupancy
// than it saves (gate_up M=8: 44.6 us staged against 22.2 us from L2).
constexpr uint32_t kXLdsBytes = 144 * 1024;
constexpr uint32_t kXLdsBytesAq4 = 64 * 1024;
#ifndef ULLM_AQ4_LDS_BATCH
#define ULLM_AQ4_LDS_BATCH 2
#endif
// Tiles per batch of the LDS-staged kernels, chosen by measurement on
// MI355X: small batches that keep a steady stream of requests in flight
// beat front-loading a wave's whole share (AQ4 M=1 4096->14336: 8.4 us at
// 2 groups per batch against 11.2 us at 8).
constexpr int kAq4LdsBatch = ULLM_AQ4_LDS_BATCH;
#ifndef ULLM_FP8_LDS_BATCH
#define ULLM_FP8_LDS_BATCH 4
#endif
constexpr int kFp8LdsBatch = ULLM_FP8_LDS_BATCH;

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
// Workgroup barrier without the memory fence of __syncthreads (which would
// drain every outstanding weight load); LDS hazards are covered by the
// explicit counter waits before it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0) only
  __builtin_amdgcn_s_barrier();
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) |
                             (0xf << 8));
}

__device__ __forceinline__ uint32_t x_slot(uint32_t r, uint32_t c,
                                           uint32_t cpr) {
  return r * cpr + (c ^ (r & 7u));
}

// Copy rows [m0, m0 + rows) of x into LDS (slot layout above) and zero one
// extra row after them; lanes whose row is past M read that zero row, so no
// A read needs masking.  Each wave DMA instruction fills 64 consecutive
// slots; lane L's slot maps back to its global chunk through the swizzle.
template <int WAVES>
__device__ __forceinline__ void stage_x_lds(const GemvArgs &a, uint16_t *xs,
                                            uint32_t rows, uint32_t cpr) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t total = rows * cpr;
  const uint32_t m0 = blockIdx.y * 32;
  for (uint32_t base = wave * kWave; base < total; base += WAVES * kWave) {
    const uint32_t p = base + lane;
    if (p < total) {
      const uint32_t r = p / cpr;
      const uint32_t c = (p % cpr) ^ (r & 7u);
      const uint16_t *src = a.x + uint64_t(m0 + r) * a.ldx + c * 8;
      __builtin_amdgcn_global_load_lds(
          (__attribute__((address_space(1))) void *)(src),
          (__attribute__((address_space(3))) void *)(xs + base * 8), 16, 0, 0);
    }
  }
  for (uint32_t c = threadIdx.x; c < cpr; c += WAVES * kWave) {
    *reinterpret_cast<u32x4 *>(xs + (total + c) * 8) = u32x4{0u, 0u, 0u, 0u};
  }
}

template <int MT, int WAVES, int B, bool FULL, int EPI>
__global__ __launch_bounds__(WAVES *kWave) void fp8_gemv_lds_kernel(
    GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  __shared__ float red[WAVES * MT * 4 * kWave];
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t T = blockIdx.x;
  const uint32_t units = a.units;
  const uint32_t ub = uint32_t(uint64_t(units) * wave / WAVES);
  const uint32_t ue = uint32_t(uint64_t(units) * (wave + 1) / WAVES);
  const u32x4 *stripe = reinterpret_cast<const u32x4 *>(
      static_cast<const uint8_t *>(a.tiles) + uint64_t(T) * units * 1024 +
      lane * 16);
  const uint32_t rows = min(32u, a.m - blockIdx.y * 32);
  const uint32_t cpr = a.k / 8;

  // Activations first (L2-resident, they land early), then the weights.
  stage_x_lds<WAVES>(a, xs, rows, cpr);
  __builtin_amdgcn_sched_barrier(0);
  const float rscale = static_cast<const float *>(a.aux)[T * 16 + threadIdx.x % 16];
  // Tile indices are clamped into [ub, ue - 1] (tile 0 for a wave with no
  // tiles) so every load stays inside this stripe.
  const uint32_t last = ue > ub ? ue - 1 : 0;
  u32x4 cur[B];
#pragma unroll
  for (int i = 0; i < B; ++i) {
    cur[i] = __builtin_nontemporal_load(stripe + uint64_t(min(ub + i, last)) * 64);
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt<B + 1>();  // this thread's activation copies have landed
  lds_barrier();

  // A operand of unit u, half h: 8 bf16 at chunk 8u + 2(lane/16) + h.
  const uint32_t cg = 2 * (lane / 16);
  const char *xa[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint32_t m = mt * 16 + lane % 16;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t r = m < rows ? m : rows;
      xa[mt][h] = reinterpret_cast<const char *>(xs) +
                  (r * cpr + ((cg + h) ^ (r & 7u))) * 16;
    }
  }
  // Four independent accumulator chains per m-tile: consecutive MFMAs never
  // wait on each other's results.
  f32x4 acc4[4][MT];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc4[c][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  for (uint32_t u = ub; u < ue; u += B) {
    u32x4 nxt[B];
    const bool more = u + B < ue;
    if (more) {
#pragma unroll
      for (int i = 0; i < B; ++i) {
        nxt[i] = __builtin_nontemporal_load(
            stripe + uint64_t(min(u + B + i, last)) * 64);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < B; ++i) {
      u32x4 wv = cur[i];
      if (!FULL) {
        const uint32_t keep = u + i < ue ? 0xffffffffu : 0u;
        wv.x &= keep;
        wv.y &= keep;
        wv.z &= keep;
        wv.w &= keep;
      }
      const u32x2 b01 = e4m3x4_to_bf16x4(wv.x);
      const u32x2 b23 = e4m3x4_to_bf16x4(wv.y);
      const u32x2 b45 = e4m3x4_to_bf16x4(wv.z);
      const u32x2 b67 = e4m3x4_to_bf16x4(wv.w);
      const bf16x8 b0 =
          __builtin_bit_cast(bf16x8, u32x4{b01.x, b01.y, b23.x, b23.y});
      const bf16x8 b1 =
          __builtin_bit_cast(bf16x8, u32x4{b45.x, b45.y, b67.x, b67.y});
      const uint32_t off = (FULL ? u + i : min(u + i, last)) * 128;
      const int ca = 2 * (i & 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const bf16x8 a0 =
            *reinterpret_cast<const bf16x8 *>(xa[mt][0] + off);
        const bf16x8 a1 =
            *reinterpret_cast<const bf16x8 *>(xa[mt][1] + off);
        acc4[ca][mt] = mfma_bf16(a0, b0, acc4[ca][mt]);
        acc4[ca + 1][mt] = mfma_bf16(a1, b1, acc4[ca + 1][mt]);
      }
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < B; ++i) {
        cur[i] = nxt[i];
      }
    }
  }
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = (acc4[0][mt] + acc4[1][mt]) + (acc4[2][mt] + acc4[3][mt]);
  }
  reduce_and_store<MT, WAVES, EPI>(a, acc, red, rscale);
}

// AQ4: the per-(row, group) activation sums sum_k x[m, k] over each 128-k
// group are formed once per workgroup in LDS, so each group costs four MFMAs
// plus one fp32 correction:
//   acc += s * (sum_k (128 + q) x  -  (128 + z) * sum_k x).
template <int MT, int WAVES, int B, bool FULL, int EPI>
__global__ __launch_bounds__(WAVES *kWave) void aq4_gemv_lds_kernel(
    GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  __shared__ float red[WAVES * MT * 4 * kWave];
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t T = blockIdx.x;
  const uint32_t groups = a.units;
  const uint32_t ub = uint32_t(uint64_t(groups) * wave / WAVES);
  const uint32_t ue = uint32_t(uint64_t(groups) * (wave + 1) / WAVES);
  const u32x4 *stripe = reinterpret_cast<const u32x4 *>(
      static_cast<const uint32_t *>(a.tiles) + uint64_t(T) * groups * 256 +
      lane * 4);
  const uint32_t *szs = static_cast<const uint32_t *>(a.aux) +
                        uint64_t(T) * groups * 16 + lane % 16;
  const uint32_t rows = min(32u, a.m - blockIdx.y * 32);
  const uint32_t cpr = a.k / 8;
  // Group sums follow the activation block and its zero row.
  float *gsum = reinterpret_cast<float *>(xs + (rows + 1) * cpr * 8);

  stage_x_lds<WAVES>(a, xs, rows, cpr);
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t last = ue > ub ? ue - 1 : 0;
  u32x4 cur[B];
  uint32_t csz[B];
#pragma unroll
  for (int i = 0; i < B; ++i) {
    const uint32_t g = min(ub + i, last);
    cur[i] = __builtin_nontemporal_load(stripe + uint64_t(g) * 64);
    csz[i] = szs[uint64_t(g) * 16];
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt<2 * B>();  // this thread's activation copies have landed
  lds_barrier();
  // 16 lanes per (row, group): lane c sums chunk c (8 values), then a
  // butterfly over the 16 lanes.  The trip count is uniform across the block.
  for (uint32_t base = 0; base < rows * groups * 16; base += WAVES * kWave) {
    const uint32_t i = base + threadIdx.x;
    const uint32_t item = i / 16, c = i % 16;
    float sum = 0.0f;
    if (item < rows * groups) {
      const uint32_t r = item / groups, g = item % groups;
      const u32x4 v =
          *reinterpret_cast<const u32x4 *>(xs + x_slot(r, g * 16 + c, cpr) * 8);
      sum = ((bits_f32(v.x << 16) + bits_f32(v.x & 0xffff0000u)) +
             (bits_f32(v.y << 16) + bits_f32(v.y & 0xffff0000u))) +
            ((bits_f32(v.z << 16) + bits_f32(v.z & 0xffff0000u)) +
             (bits_f32(v.w << 16) + bits_f32(v.w & 0xffff0000u)));
    }
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) {
      sum += __shfl_xor(sum, off, kWave);
    }
    if (item < rows * groups && c == 0) {
      gsum[item] = sum;
    }
  }
  lds_barrier();

  // A operand of group g, MFMA j: chunk 16g + (lane/16) + 4j of row m.
  const uint32_t q4 = lane / 16;
  const char *xa[MT][4];
  const float *gs[MT][4];  // group-sum row of each accumulator element
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint32_t m = mt * 16 + lane % 16;
    const uint32_t r = m < rows ? m : rows;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xa[mt][j] = reinterpret_cast<const char *>(xs) +
                  (r * cpr + ((q4 + 4 * j) ^ (r & 7u))) * 16;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t mr = mt * 16 + 4 * q4 + e;
      gs[mt][e] = gsum + (mr < rows ? mr : 0) * groups;
    }
  }
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t nmask = opaque_u32(0x000f000fu);
  const uint32_t nmagic = opaque_u32(0x43004300u);

  for (uint32_t g = ub; g < ue; g += B) {
    u32x4 nxt[B];
    uint32_t nsz[B];
    const bool more = g + B < ue;
    if (more) {
#pragma unroll
      for (int i = 0; i < B; ++i) {
        const uint32_t gg = min(g + B + i, last);
        nxt[i] = __builtin_nontemporal_load(stripe + uint64_t(gg) * 64);
        nsz[i] = szs[uint64_t(gg) * 16];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // The batch's groups are independent MFMA chains; issuing them
    // interleaved (j outer, group inner) hides the accumulate latency.
    f32x4 p[B][MT];
#pragma unroll
    for (int i = 0; i < B; ++i) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        p[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < B; ++i) {
        const bf16x8 bj = nib8_to_bf16_off128(cur[i][j], nmask, nmagic);
        const uint32_t off = (FULL ? g + i : min(g + i, last)) * 256;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          p[i][mt] = mfma_bf16(*reinterpret_cast<const bf16x8 *>(xa[mt][j] + off),
                               bj, p[i][mt]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < B; ++i) {
      // A clamped (repeated) tile contributes zero through its scale.
      const float sf = (FULL || g + i < ue)
                           ? f16_to_f32(uint16_t(csz[i] & 0xffffu))
                           : 0.0f;
      const float zoff = 128.0f + f16_to_f32(uint16_t(csz[i] >> 16));
      const uint32_t gi = FULL ? g + i : min(g + i, last);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[mt][r] += sf * (p[i][mt][r] - zoff * gs[mt][r][gi]);
        }
      }
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < B; ++i) {
        cur[i] = nxt[i];
        csz[i] = nsz[i];
      }
    }
  }
  reduce_and_store<MT, WAVES, EPI>(a, acc, red, 1.0f);
}

// Cross-wave reduction of one stripe for the multi-stripe kernels: like
// reduce_and_store, but for stripe T, through one of two LDS buffers that
// alternate between stripes, and behind a barrier that leaves the weight
// loads already issued for the next stripe in flight.
template <int MT, int WAVES, int EPI = kEpiNone>
__device__ __forceinline__ void flush_stripe(const GemvArgs &a,
                                             f32x4 (&acc)[MT], float *red,
                                             uint32_t T, float scale) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      red[((wave * MT + mt) * 4 + r) * kWave + lane] = acc[mt][r];
    }
  }
  lds_barrier();
  const uint32_t m_base = blockIdx.y * 32;
  for (int o = threadIdx.x; o < MT * 256; o += WAVES * kWave) {
    const int mt = o / 256;
    const int mrow = (o % 256) / 16;
    const int ncol = o % 16;
    const int src_lane = ncol + 16 * (mrow / 4);
    const int r = mrow % 4;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      v += red[((w * MT + mt) * 4 + r) * kWave + src_lane];
    }
    const uint32_t m = m_base + mt * 16 + mrow;
    const uint32_t n = T * 16 + ncol;
    store_out<EPI>(a.y, a.ldy, a.y_f32, a.epi, a.n, m, n, a.alpha * (scale * v),
              m < a.m);
  }
}


// Activation block layout of the multi-stripe kernels: row r's 16-byte
// chunk c at slot r * (cpr + 1) + c.  The one-chunk row padding puts the 16
// rows an MFMA A read touches (same chunk, consecutive rows) in 16 different
// bank groups, and every chunk of a lane sits at a fixed offset from the
// lane's row base, so A reads need no per-read address arithmetic.  Row
// `rows` is all zero; lanes whose row is past M read it.
template <int WAVES>
__device__ __forceinline__ void stage_x_pad(const GemvArgs &a, uint16_t *xs,
                                            uint32_t rows, uint32_t cpr) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t pitch = cpr + 1;
  const uint32_t total = rows * pitch;
  const uint32_t m0 = blockIdx.y * 32;
  for (uint32_t base = wave * kWave; base < total; base += WAVES * kWave) {
    const uint32_t p = base + lane;
    const uint32_t r = p / pitch, c = p % pitch;
    if (p < total && c < cpr) {
      const uint16_t *src = a.x + uint64_t(m0 + r) * a.ldx + c * 8;
      __builtin_amdgcn_global_load_lds(
          (__attribute__((address_space(1))) void *)(src),
          (__attribute__((address_space(3))) void *)(xs + base * 8), 16, 0, 0);
    }
  }
  for (uint32_t c = threadIdx.x; c < cpr; c += WAVES * kWave) {
    *reinterpret_cast<u32x4 *>(xs + (total + c) * 8) = u32x4{0u, 0u, 0u, 0u};
  }
}

// LDS bytes of the multi-stripe kernels: padded activation rows and the zero
// row.
uint32_t ms_lds_bytes(const GemvArgs &a) {
  const uint32_t rows = min(a.m, 32u);
  return (rows + 1) * (a.k * 2 + 16);
}

// End of one stripe for the multi-stripe kernels, for the KS waves that
// split its K: with KS = 1 each lane stores its accumulators directly (lane
// l holds rows 4 (l / 16) + r, column l % 16 of every 16 x 16 tile); with
// KS > 1 the partial sums meet in LDS behind a workgroup barrier that does
// not wait on vector loads (the next stripe's weights stay in flight), and
// the sub-group's threads store.  `red` is this sub-group's buffer, `kw` the
// wave's index within it, `live` whether the stripe exists.
template <int MT, int KS, int P = 1, int ROWS = 16, int EPI = kEpiNone>
__device__ __forceinline__ void flush_ks(const GemvArgs &a, f32x4 (&acc)[MT],
                                         float *red, uint32_t T, float scale,
                                         uint32_t kw, bool live) {
  // P = 4: the four classes (lane groups l / 16) are summed in registers
  // first, leaving every lane with the full sum of rows 0..3; only the first
  // ROWS rows are stored.
  static_assert(P == 1 || (P == 4 && MT == 1 && ROWS <= 4), "packing");
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t m_base = blockIdx.y * 32;
  // Called by every lane of the wave (the epilogue pairs lanes l, l ^ 8).
  auto store = [&](uint32_t m, uint32_t n, float v, bool ok) {
    store_out<EPI>(a.y, a.ldy, a.y_f32, a.epi, a.n, m, n, a.alpha * (scale * v),
              ok && live && m < a.m);
  };
  if constexpr (P == 4) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      acc[0][r] += __shfl_xor(acc[0][r], 16, kWave);
      acc[0][r] += __shfl_xor(acc[0][r], 32, kWave);
    }
  }
  if constexpr (KS == 1 && P == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        store(m_base + mt * 16 + 4 * (lane / 16) + r, T * 16 + lane % 16,
              acc[mt][r], true);
      }
    }
  } else if constexpr (KS == 1) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      // Every lane holds the class sum; lanes 0..15 store it.
      store(m_base + r, T * 16 + lane % 16, acc[0][r], lane < 16);
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        red[((kw * MT + mt) * 4 + r) * kWave + lane] = acc[mt][r];
      }
    }
    lds_barrier();
    for (uint32_t o = kw * kWave + lane; o < MT * ROWS * 16; o += KS * kWave) {
      const uint32_t mt = o / (ROWS * 16), mrow = (o % (ROWS * 16)) / 16;
      const uint32_t ncol = o % 16;
      // P = 4: row mrow's class sum sits in element mrow of lanes 0..15.
      const uint32_t src = P == 1 ? ncol + 16 * (mrow / 4) : ncol;
      const uint32_t r = mrow % 4;
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < KS; ++w) {
        v += red[((w * MT + mt) * 4 + r) * kWave + src];
      }
      store(m_base + mt * 16 + mrow, T * 16 + ncol, v, true);
    }
  }
}

// Multi-stripe AQ4 kernel (M <= 4).  A workgroup stages its activation block
// in LDS once and then works through a run of a.spw consecutive stripes.  Its WAVES waves form WAVES / KS sub-groups; sub-group g takes
// stripes g, g + WAVES / KS, ... of the run, and its KS waves split each
// stripe's K (KS = 1: a wave owns whole stripes and needs no reduction).
// Each wave's weight stream is one software pipeline over all its stripes: a
// ring of DEPTH batch buffers keeps DEPTH - 1 batches in flight while one is
// contracted, also across the per-stripe reduction.  Loop bounds are
// wave-uniform scalars and look-ahead loads are unconditional (past the run,
// or for a sub-group's missing last stripe, they read zeros from outside the
// buffer range without touching memory), so no wait on outstanding loads is
// forced before the data is used; the tile offset is a scalar operand of the
// buffer load.
// NR: accumulator elements that can hold a valid row (only rows r < NR <= M
// carry results and need the per-group correction).
// Requires groups % (KS * B) == 0 (every wave's share is whole batches).
//
// The A operand rows are packed in four classes of four, as in the
// register-staged kernels: class c of the single A read of a group
// holds the activation rows for the group's 32-k block c, so one ones-MFMA
// gives every class its block's activation sum and the per-(row, group) sums
// need no separate pass over LDS (the pass and its barrier sat between the
// arrival of x and the first MFMA: 0.8 us of the M=1 4096->14336 launch on
// MI355X).  Block c's product is valid in class c's rows only; each lane
// keeps its own class's, and the classes are summed at the stripe's end.
template <int WAVES, int KS, int B, int DEPTH, int NR, int EPI>
__global__ __launch_bounds__(WAVES *kWave) void aq4_gemv_ms_kernel(
    GemvArgs a) {
  static_assert(NR >= 1 && NR <= 4, "rows of one class");
  static_assert(WAVES % KS == 0, "sub-groups");
  constexpr int MT = 1, P = 4;
  constexpr uint32_t SG = WAVES / KS;
  constexpr uint32_t RED = KS > 1 ? 2 * WAVES * MT * 4 * kWave : 1;
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  __shared__ float red[RED];
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t sg = wave / KS, kw = wave % KS;
  const uint32_t groups = a.units;
  const uint32_t stripes = a.n16 / 16;
  const uint32_t T0 = blockIdx.x * a.spw;
  const uint32_t nS = min(a.spw, stripes - T0);
  const uint32_t per_sg = (nS + SG - 1) / SG;  // stripes per sub-group (uniform)
  const uint32_t ub = groups * kw / KS;
  const uint32_t ue = groups * (kw + 1) / KS;
  const uint32_t nbw = (ue - ub) / B;  // batches per stripe
  const uint32_t NB = per_sg * nbw;    // batches of this wave
  const __amdgpu_buffer_rsrc_t wbuf = byte_buffer(
      static_cast<const uint8_t *>(a.tiles) + uint64_t(T0) * groups * 1024,
      nS * groups * 1024);
  const __amdgpu_buffer_rsrc_t zbuf = byte_buffer(
      static_cast<const uint32_t *>(a.aux) + uint64_t(T0) * groups * 16,
      nS * groups * 64);
  const uint32_t wlane = lane * 16, zlane = (lane % 16) * 4;
  const uint32_t rows = min(32u, a.m - blockIdx.y * 32);
  const uint32_t cpr = a.k / 8;
  const uint32_t pitch = cpr + 1;

  struct Batch {
    u32x4 w[B];
    uint32_t sz[B];
  };
  // Load pointer: the wave's ls-th stripe (run stripe sg + ls * SG), group
  // lg (scalars).
  uint32_t ls = 0, lg = ub;
  auto issue = [&](Batch &bt) {
    const uint32_t item = (sg + ls * SG) * groups + lg;
#pragma unroll
    for (int i = 0; i < B; ++i) {
      bt.w[i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     wbuf, wlane, (item + i) * 1024, kNt));
      bt.sz[i] = __builtin_amdgcn_raw_buffer_load_b32(zbuf, zlane,
                                                      (item + i) * 64, 0);
    }
    lg += B;
    if (lg == ue) {
      lg = ub;
      ++ls;
    }
  };

  stage_x_pad<WAVES>(a, xs, rows, cpr);
  __builtin_amdgcn_sched_barrier(0);
  Batch ring[DEPTH];
#pragma unroll
  for (int r = 0; r + 1 < DEPTH; ++r) {
    issue(ring[r]);
    // Keep the batches in ring order: the steady-state waits assume that
    // batch r's loads are all older than batch r + 1's.
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_vmcnt<(DEPTH - 1) * 2 * B>();  // this thread's activation copies landed
  lds_barrier();

  // A operand of group g: lane l reads row l % 4 of class (l % 16) / 4,
  // i.e. chunk 16 g + 4 ((l % 16) / 4) + l / 16 of that row (rows past M
  // read the zero row).
  const char *xa;
  {
    const uint32_t m = lane % 4;
    const uint32_t r = m < rows ? m : rows;
    xa = reinterpret_cast<const char *>(xs) +
         (r * pitch + 4u * ((lane % 16) / 4) + lane / 16) * 16;
  }
  const uint32_t nmask = opaque_u32(0x000f000fu);
  const uint32_t nmagic = opaque_u32(0x43004300u);
  const bf16x8 ones = __builtin_bit_cast(
      bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
  // Class of this lane's rows: lane / 16.
  const bool odd = (lane / 16) & 1u, high = (lane / 32) & 1u;

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // Consume pointer: the wave's cs-th stripe, group cg.
  uint32_t cs = 0, cg = ub;
  auto consume = [&](const Batch &bt) {
    f32x4 xsum[B], p[B][4];
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const bf16x8 xa0 =
          *reinterpret_cast<const bf16x8 *>(xa + (cg + i) * 256);
      xsum[i] = mfma_bf16(xa0, ones, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        p[i][c] = mfma_bf16(xa0, nib8_to_bf16_off128(bt.w[i][c], nmask, nmagic),
                            f32x4{0.f, 0.f, 0.f, 0.f});
      }
    }
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const float sf = f16_to_f32(uint16_t(bt.sz[i] & 0xffffu));
      const float zoff = 128.0f + f16_to_f32(uint16_t(bt.sz[i] >> 16));
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        // Two-level select on the lane's class bits, element by element (a
        // select over the whole p[i][.] array compiled to a dynamically
        // indexed stack copy).
        const float q01 = odd ? p[i][1][r] : p[i][0][r];
        const float q23 = odd ? p[i][3][r] : p[i][2][r];
        const float q = high ? q23 : q01;
        acc[0][r] += sf * (q - zoff * xsum[i][r]);
      }
    }
    cg += B;
    if (cg == ue) {  // stripe done: reduce, store, reset
      const uint32_t sr = sg + cs * SG;  // run stripe
      flush_ks<MT, KS, P, NR, EPI>(a, acc,
                          red + (cs & 1) * (RED / 2) + sg * KS * MT * 4 * kWave,
                          T0 + sr, 1.0f, kw, sr < nS);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      cg = ub;
      ++cs;
    }
  };

  // Ring of DEPTH batch buffers; indices are compile-time, so the ring lives
  // in registers.
  for (uint32_t t = 0; t < NB; t += DEPTH) {
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) {
      issue(ring[(r + DEPTH - 1) % DEPTH]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + r < NB) {
        consume(ring[r]);
      }
    }
  }
}

// Multi-stripe FP8 kernel: the AQ4 multi-stripe kernel's structure (x staged
// once per workgroup in the padded layout, a run of a.spw stripes, one ring
// pipeline per wave over the run) with 64-k FP8 units.  Each batch also
// carries the row scales of its stripe, applied once in the per-stripe
// reduction.  Requires units % (WAVES * B) == 0.
template <int MT, int WAVES, int B, int DEPTH, int EPI>
__global__ __launch_bounds__(WAVES *kWave) void fp8_gemv_ms_kernel(
    GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  __shared__ float red[2][WAVES * MT * 4 * kWave];
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t units = a.units;
  const uint32_t stripes = a.n16 / 16;
  const uint32_t T0 = blockIdx.x * a.spw;
  const uint32_t nS = min(a.spw, stripes - T0);
  const uint32_t ub = units * wave / WAVES;
  const uint32_t ue = units * (wave + 1) / WAVES;
  const uint32_t nbw = (ue - ub) / B;
  const uint32_t NB = nS * nbw;
  const __amdgpu_buffer_rsrc_t wbuf = byte_buffer(
      static_cast<const uint8_t *>(a.tiles) + uint64_t(T0) * units * 1024,
      nS * units * 1024);
  const __amdgpu_buffer_rsrc_t sbuf = byte_buffer(
      static_cast<const float *>(a.aux) + uint64_t(T0) * 16, nS * 64);
  const uint32_t wlane = lane * 16, slane = (lane % 16) * 4;
  const uint32_t rows = min(32u, a.m - blockIdx.y * 32);
  const uint32_t cpr = a.k / 8;
  const uint32_t pitch = cpr + 1;

  struct Batch {
    u32x4 w[B];
    float rs;  // row scale of the batch's stripe (column lane % 16)
  };
  uint32_t ls = 0, lu = ub;
  auto issue = [&](Batch &bt) {
    const uint32_t item = ls * units + lu;
#pragma unroll
    for (int i = 0; i < B; ++i) {
      bt.w[i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     wbuf, wlane, (item + i) * 1024, kNt));
    }
    bt.rs = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(sbuf, slane, ls * 64, 0));
    lu += B;
    if (lu == ue) {
      lu = ub;
      ++ls;
    }
  };

  stage_x_pad<WAVES>(a, xs, rows, cpr);
  __builtin_amdgcn_sched_barrier(0);
  Batch ring[DEPTH];
#pragma unroll
  for (int r = 0; r + 1 < DEPTH; ++r) {
    issue(ring[r]);
    // Keep the batches in ring order: the steady-state waits assume that
    // batch r's loads are all older than batch r + 1's.
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_vmcnt<(DEPTH - 1) * (B + 1)>();  // this thread's activation copies landed
  lds_barrier();

  // A operand of unit u, half h: chunk 8 u + 2 (lane / 16) + h of the row.
  const char *xa[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint32_t m = mt * 16 + lane % 16;
    const uint32_t r = m < rows ? m : rows;
    xa[mt] = reinterpret_cast<const char *>(xs) +
             (r * pitch + 2 * (lane / 16)) * 16;
  }
  f32x4 acc4[4][MT];
  auto zero_acc = [&]() {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc4[c][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  zero_acc();
  uint32_t cs = 0, cu = ub;
  auto consume = [&](const Batch &bt) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const u32x4 wv = bt.w[i];
      const u32x2 b01 = e4m3x4_to_bf16x4(wv.x);
      const u32x2 b23 = e4m3x4_to_bf16x4(wv.y);
      const u32x2 b45 = e4m3x4_to_bf16x4(wv.z);
      const u32x2 b67 = e4m3x4_to_bf16x4(wv.w);
      const bf16x8 w0 =
          __builtin_bit_cast(bf16x8, u32x4{b01.x, b01.y, b23.x, b23.y});
      const bf16x8 w1 =
          __builtin_bit_cast(bf16x8, u32x4{b45.x, b45.y, b67.x, b67.y});
      const uint32_t off = (cu + i) * 128;
      const int ca = 2 * (i & 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc4[ca][mt] = mfma_bf16(
            *reinterpret_cast<const bf16x8 *>(xa[mt] + off), w0, acc4[ca][mt]);
        acc4[ca + 1][mt] = mfma_bf16(
            *reinterpret_cast<const bf16x8 *>(xa[mt] + off + 16), w1,
            acc4[ca + 1][mt]);
      }
    }
    cu += B;
    if (cu == ue) {
      f32x4 acc[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = (acc4[0][mt] + acc4[1][mt]) + (acc4[2][mt] + acc4[3][mt]);
      }
      flush_stripe<MT, WAVES, EPI>(a, acc, red[cs & 1], T0 + cs, bt.rs);
      zero_acc();
      cu = ub;
      ++cs;
    }
  };

  for (uint32_t t = 0; t < NB; t += DEPTH) {
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) {
      issue(ring[(r + DEPTH - 1) % DEPTH]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + r < NB) {
        consume(ring[r]);
      }
    }
  }
}

// Split K.  With few stripes and a long K, the register-staged kernels split
// each stripe group's K over a.ksplit workgroups (so that groups of S
// stripes, which share their activation loads, still fill the chip).  Each
// workgroup writes its fp32 partial sums to a.part; the last of the ksplit
// workgroups to arrive at the group's counter adds them in fixed order
// (deterministic) and stores the output.  No workgroup waits for another:
// the counter only elects the finisher, which also resets it to zero for the
// next call.  Partial slot of (k part, stripe T, row, column):
// ((kp * stripes + T) * rows + row) * 16 + column, rows = MT * 16.
//
// The workgroups of a group may sit on different XCDs, whose L2 caches are
// not coherent with each other.  Instead of device-scope fences (each one
// writes back or invalidates a whole L2), the partial sums are stored and
// loaded with the system-coherent cache policy (sc0 sc1), which goes to
// memory, and the counter is a device-scope atomic issued after this
// workgroup's stores have completed.
//
// Why this is ordered without release/acquire fences (the gfx942/gfx950
// memory model of the LLVM AMDGPU backend, which maps an agent-scope release
// store to "buffer_wbl2 sc1; s_waitcnt vmcnt(0); store sc1" and an
// agent-scope acquire load to "load sc1; s_waitcnt vmcnt(0); buffer_inv sc1"):
//   * the L2 write-back of the release exists to push this XCD's dirty lines
//     to memory; the partial sums are never dirty in L2, because sc0 sc1
//     stores write through to memory, and s_waitcnt vmcnt(0) (below) returns
//     only once every one of them is acknowledged by memory, which is the
//     ordering the release's wait provides;
//   * the agent-scope atomic (sc1) is performed at memory, after those
//     acknowledgements, so the workgroup that reads count ks - 1 from it
//     runs after every other workgroup's partial stores reached memory;
//   * the L2 invalidate of the acquire exists so that later plain loads
//     cannot hit stale lines of this XCD's L2; the finisher's partial loads
//     are sc0 sc1 loads, which are served from memory, not from a possibly
//     stale L2 line.
// The finisher then adds the parts in k order, so results are deterministic.
constexpr int kSc = 1 | 16;  // sc0 | sc1

// Element i of the partial sums through a buffer descriptor over a.part
// (the scratch stays below 2 GiB).
__device__ __forceinline__ void sk_put(__amdgpu_buffer_rsrc_t part, uint64_t i, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), part,
                                        uint32_t(i * 4), 0, kSc);
}
__device__ __forceinline__ float sk_get(__amdgpu_buffer_rsrc_t part, uint64_t i) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(part, uint32_t(i * 4), 0, kSc));
}

__device__ __forceinline__ bool sk_arrive(uint32_t *cnt, uint32_t ks,
                                          uint32_t *flag) {
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores completed
  lds_barrier();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev + 1 == ks;
    if (last) {
      __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    *flag = last ? 1u : 0u;
  }
  lds_barrier();
  return *flag != 0;
}

// Register-staged multi-stripe FP8 kernel, for activation blocks too large
// for LDS (M > 16 at K = 4096, or long K).  Each wave reads its K share of
// the activations straight from L2 into registers and reuses them across S
// adjacent stripes ("stripe group"), so x is read from L2 once per S stripes
// instead of once per stripe; a workgroup walks a run of a.spw stripe groups
// with its WAVES waves splitting K, one ring pipeline per wave (weights, x
// and the row scales of a batch travel together), and the partial sums of a
// stripe group meet in LDS.  Rows past M are read at an offset outside the
// activation buffer (zeros, no memory access).  Requires units % (WAVES * B)
// == 0.  P = 2 packs the two 32-k blocks of a unit into one activation load
// for M <= 8, as described at the AQ4 register-staged kernel; the two block
// products accumulate separately and each lane keeps its own class's.
template <int MT, int WAVES, int S, int B, int DEPTH, int P, int EPI, bool SK>
__global__ __launch_bounds__(WAVES *kWave) void fp8_gemv_rs_kernel(
    GemvArgs a) {
  static_assert(P == 1 || (P == 2 && MT == 1), "row packing: one m-tile");
  constexpr int XR = 2 / P;            // activation registers per unit
  constexpr uint32_t RP = 16 / P;      // rows per class
  __shared__ float red[2][WAVES * S * MT * 4 * kWave];
  __shared__ uint32_t sk_flag;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t units = a.units;
  const uint32_t stripes = a.n16 / 16;
  const uint32_t G = (stripes + S - 1) / S;  // stripe groups
  // Split K: workgroup kp of a group's a.ksplit streams K part kp.
  const uint32_t ks = SK ? a.ksplit : 1u;
  const uint32_t kp = SK ? blockIdx.x % ks : 0u;
  const uint32_t G0 = (SK ? blockIdx.x / ks : blockIdx.x) * a.spw;
  const __amdgpu_buffer_rsrc_t pbuf = byte_buffer(a.part, 0x7ffffff0u);
  const uint32_t nG = min(a.spw, G - G0);
  const uint32_t T0 = G0 * S;
  const uint32_t nT = min(nG * S, stripes - T0);  // stripes of the run
  const uint32_t upk = units / ks;  // units of a K part
  const uint32_t ub = kp * upk + upk * wave / WAVES;
  const uint32_t ue = kp * upk + upk * (wave + 1) / WAVES;
  const uint32_t nbw = (ue - ub) / B;
  const uint32_t NB = nG * nbw;
  const __amdgpu_buffer_rsrc_t wbuf = byte_buffer(
      static_cast<const uint8_t *>(a.tiles) + uint64_t(T0) * units * 1024,
      nT * units * 1024);
  const __amdgpu_buffer_rsrc_t sbuf = byte_buffer(
      static_cast<const float *>(a.aux) + uint64_t(T0) * 16, nT * 64);
  const uint32_t m0 = blockIdx.y * 32;
  const uint32_t rows = min(32u, a.m - m0);
  const __amdgpu_buffer_rsrc_t xbuf = byte_buffer(
      a.x + uint64_t(m0) * a.ldx, uint32_t(((rows - 1) * a.ldx + a.k) * 2));
  // MFMA lane 16 h + r of register t takes A row r and the 16 bytes at
  // chunk 2 h + t (P = 1; row r = m) or 2 h + c (P = 2; row r = 8 c + m) of
  // the unit's 128-byte row segment.  The loads read whole row segments
  // instead, 8 lanes per row (lane 8 m' + j reads chunk j of row m', rows
  // 8 u .. 8 u + 7 in register u), so a lane quad reads one contiguous 64
  // bytes, which the texture path serves as one access instead of four; a
  // lane permute (xperm) then hands each lane its MFMA operand.
  // The split-K launches (long K, 9 <= M <= 32) keep the MFMA-order loads:
  // with two m-tiles the permutes cost more than they save there (MI355X,
  // FP8 M=32 14336->4096: 2.33 against 2.53 TB/s).
  constexpr bool XP = !SK;
  uint32_t xoff[MT][XR];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int u = 0; u < XR; ++u) {
      if constexpr (XP) {
        const uint32_t m = mt * 16 + 8 * u + lane / 8;
        xoff[mt][u] = m < rows ? uint32_t((m * a.ldx) * 2 + 16 * (lane % 8))
                               : 0x80000000u;
      } else {
        const uint32_t m = mt * 16 + (lane % 16) % RP;
        const uint32_t c = (lane % 16) / RP;
        xoff[mt][u] = m < rows ? uint32_t((m * a.ldx + 16 * (lane / 16)) * 2 +
                                          16 * c + 16 * u)
                               : 0x80000000u;
      }
    }
  }
  // Source lane (bpermute byte address) of MFMA lane 16 h + r.
  const uint32_t xh = lane / 16, xr = lane % 16;
  const int xsrc0 = P == 2 ? int((8 * (xr % 8) + 2 * xh + xr / 8) * 4)
                           : int((8 * (xr % 8) + 2 * xh) * 4);
  const int xsrc1 = xsrc0 + 4;  // P = 1, register t = 1: chunk 2 h + 1
  const bool xlo = xr < 8;      // P = 1: rows 0..7 come from register 0
  auto xperm = [&](const bf16x8 (&v)[XR], int t) {
    if constexpr (!XP) {
      return v[t];
    }
    const int src = t == 0 ? xsrc0 : xsrc1;
    u32x4 o;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int lo = __builtin_amdgcn_ds_bpermute(
          src, int(__builtin_bit_cast(u32x4, v[0])[d]));
      if constexpr (XR == 2) {
        const int hi = __builtin_amdgcn_ds_bpermute(
            src, int(__builtin_bit_cast(u32x4, v[XR - 1])[d]));
        o[d] = uint32_t(xlo ? lo : hi);
      } else {
        o[d] = uint32_t(lo);
      }
    }
    return __builtin_bit_cast(bf16x8, o);
  };
  const uint32_t lcls = (lane / 16) * 4 / RP;
  const uint32_t wlane = lane * 16, slane = (lane % 16) * 4;

  struct Batch {
    u32x4 w[B][S];
    bf16x8 x[B][MT][XR];
    float rs[S];
  };
  // Load pointer: stripe group lg of the run, unit lu (scalars).  Past the
  // run the weight and scale loads fall outside their buffers and the
  // activation loads are pushed outside theirs, so they read zeros.
  uint32_t lg = 0, lu = ub;
  auto issue = [&](Batch &bt) {
    const uint32_t xpast = lg < nG ? 0u : 0x80000000u;
#pragma unroll
    for (int i = 0; i < B; ++i) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int t = 0; t < XR; ++t) {
          bt.x[i][mt][t] = __builtin_bit_cast(
              bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                          xbuf, xoff[mt][t], ((lu + i) * 128) | xpast, 0));
        }
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        bt.w[i][s] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       wbuf, wlane, ((lg * S + s) * units + lu + i) * 1024, kNt));
      }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      bt.rs[s] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(sbuf, slane,
                                                      (lg * S + s) * 64, 0));
    }
    lu += B;
    if (lu == ue) {
      lu = ub;
      ++lg;
    }
  };

  Batch ring[DEPTH];
#pragma unroll
  for (int r = 0; r + 1 < DEPTH; ++r) {
    issue(ring[r]);
    // Keep the batches in ring order: the steady-state waits assume that
    // batch r's loads are all older than batch r + 1's.
    __builtin_amdgcn_sched_barrier(0);
  }
  f32x4 acc[S][MT][P];
  auto zero_acc = [&]() {
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int c = 0; c < P; ++c) {
          acc[s][mt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  };
  zero_acc();
  uint32_t cgp = 0, cu = ub;
  auto consume = [&](const Batch &bt) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      bf16x8 xv[MT][XR];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int t = 0; t < XR; ++t) {
          xv[mt][t] = xperm(bt.x[i][mt], t);
        }
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const u32x4 wv = bt.w[i][s];
        const u32x2 b01 = e4m3x4_to_bf16x4(wv.x);
        const u32x2 b23 = e4m3x4_to_bf16x4(wv.y);
        const u32x2 b45 = e4m3x4_to_bf16x4(wv.z);
        const u32x2 b67 = e4m3x4_to_bf16x4(wv.w);
        const bf16x8 w0 =
            __builtin_bit_cast(bf16x8, u32x4{b01.x, b01.y, b23.x, b23.y});
        const bf16x8 w1 =
            __builtin_bit_cast(bf16x8, u32x4{b45.x, b45.y, b67.x, b67.y});
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[s][mt][0] = mfma_bf16(xv[mt][0], w0, acc[s][mt][0]);
          acc[s][mt][P - 1] = mfma_bf16(xv[mt][XR - 1], w1, acc[s][mt][P - 1]);
        }
      }
    }
    cu += B;
    if (cu == ue) {  // stripe group done: reduce across waves, store, reset
      float *rb = red[cgp & 1];
#pragma unroll
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x4 q = P == 1 || lcls == 0 ? acc[s][mt][0] : acc[s][mt][P - 1];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            rb[(((wave * S + s) * MT + mt) * 4 + r) * kWave + lane] = q[r];
          }
        }
      }
      lds_barrier();
      const uint32_t Tg = T0 + cgp * S;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        for (uint32_t o = threadIdx.x; o < MT * RP * 16; o += WAVES * kWave) {
          const uint32_t mt = o / (RP * 16), mrow = (o % (RP * 16)) / 16;
          const uint32_t ncol = o % 16;
          float v = 0.0f;
#pragma unroll
          for (int c = 0; c < P; ++c) {
            const uint32_t arow = c * RP + mrow;
            const uint32_t src = ncol + 16 * (arow / 4), r = arow % 4;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
              v += rb[(((w * S + s) * MT + mt) * 4 + r) * kWave + src];
            }
          }
          const uint32_t m = m0 + mt * 16 + mrow, n = (Tg + s) * 16 + ncol;
          if constexpr (SK) {
            // A ragged last group's missing stripes have no slot (slot
            // stripes would alias the next K part's stripe 0).
            if (Tg + s < stripes) {
              sk_put(pbuf,
                     ((uint64_t(kp) * stripes + Tg + s) * (MT * 16) + mt * 16 + mrow) * 16 +
                         ncol,
                     v);
            }
          } else {
            store_out<EPI>(a.y, a.ldy, a.y_f32, a.epi, a.n, m, n,
                    a.alpha * (bt.rs[s] * v), m < a.m);
          }
        }
      }
      if constexpr (SK) {
        if (sk_arrive(a.cnt + G0 + cgp, ks, &sk_flag)) {
#pragma unroll
          for (int s = 0; s < S; ++s) {
            if (Tg + s >= stripes) {
              break;
            }
            for (uint32_t o = threadIdx.x; o < MT * RP * 16; o += WAVES * kWave) {
              const uint32_t mt = o / (RP * 16), mrow = (o % (RP * 16)) / 16;
              const uint32_t ncol = o % 16;
              float v = 0.0f;
              for (uint32_t k = 0; k < ks; ++k) {
                v += sk_get(pbuf, ((uint64_t(k) * stripes + Tg + s) * (MT * 16) +
                                     mt * 16 + mrow) * 16 + ncol);
              }
              const uint32_t m = m0 + mt * 16 + mrow, n = (Tg + s) * 16 + ncol;
              store_out<EPI>(a.y, a.ldy, a.y_f32, a.epi, a.n, m, n,
                    a.alpha * (bt.rs[s] * v), m < a.m);
            }
          }
        }
      }
      zero_acc();
      cu = ub;
      ++cgp;
    }
  };

  for (uint32_t t = 0; t < NB; t += DEPTH) {
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) {
      issue(ring[(r + DEPTH - 1) % DEPTH]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + r < NB) {
        consume(ring[r]);
      }
    }
  }
}

// Register-staged multi-stripe AQ4 kernel: the FP8 register-staged kernel's
// structure with 128-k groups.  Each wave reads its K share of x from L2
// into registers once per group of S adjacent stripes; the per-group
// activation sums come from one MFMA against a ones operand, shared by the S
// stripes.  Requires groups % (WAVES * B) == 0.
//
// Row packing (P = 2 or 4, one m-tile, M <= 16 / P): the 16 A rows of an
// MFMA are split into P classes of 16 / P rows, and class c of x register t
// holds the activation rows for 32-k block P t + c of the group.  One 16-byte
// activation load then carries P blocks instead of one, which matters
// because the texture path charges every activation load for 64 lanes
// whether or not their rows exist (AQ4 M=8 14336->4096 on MI355X: 12.8 us
// with four activation loads per group, 8.3 us in a timing-only variant that
// issued one).  The product of
// register t with block P t + c's weights is valid only in class c's rows,
// so the P block products go to separate accumulators p[c] and each lane
// keeps the one of its own class (a lane's four accumulator rows lie in one
// class); the class rows of a stripe are summed in the final reduction.  The
// ones-MFMA of register t gives every class the sum over its own blocks, so
// a group needs 4 / P sum MFMAs instead of 4.
template <int MT, int WAVES, int S, int B, int DEPTH, int P, int EPI, bool SK>
__global__ __launch_bounds__(WAVES *kWave) void aq4_gemv_rs_kernel(
    GemvArgs a) {
  static_assert(P == 1 || MT == 1, "row packing needs a single m-tile");
  static_assert(P == 1 || P == 2 || P == 4, "P divides the 4 blocks of a group");
  constexpr int XR = 4 / P;            // activation registers per group
  constexpr uint32_t RP = 16 / P;      // rows per class
  __shared__ float red[2][WAVES * S * MT * 4 * kWave];
  __shared__ uint32_t sk_flag;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t groups = a.units;
  const uint32_t stripes = a.n16 / 16;
  const uint32_t G = (stripes + S - 1) / S;  // stripe groups
  // Split K: workgroup kp of a group's a.ksplit streams K part kp.
  const uint32_t ks = SK ? a.ksplit : 1u;
  const uint32_t kp = SK ? blockIdx.x % ks : 0u;
  const uint32_t G0 = (SK ? blockIdx.x / ks : blockIdx.x) * a.spw;
  const __amdgpu_buffer_rsrc_t pbuf = byte_buffer(a.part, 0x7ffffff0u);
  const uint32_t nG = min(a.spw, G - G0);
  const uint32_t T0 = G0 * S;
  const uint32_t nT = min(nG * S, stripes - T0);
  const uint32_t upk = groups / ks;  // units of a K part
  const uint32_t ub = kp * upk + upk * wave / WAVES;
  const uint32_t ue = kp * upk + upk * (wave + 1) / WAVES;
  const uint32_t nbw = (ue - ub) / B;
  const uint32_t NB = nG * nbw;
  const __amdgpu_buffer_rsrc_t wbuf = byte_buffer(
      static_cast<const uint8_t *>(a.tiles) + uint64_t(T0) * groups * 1024,
      nT * groups * 1024);
  const __amdgpu_buffer_rsrc_t zbuf = byte_buffer(
      static_cast<const uint32_t *>(a.aux) + uint64_t(T0) * groups * 16,
      nT * groups * 64);
  const uint32_t m0 = blockIdx.y * 32;
  const uint32_t rows = min(32u, a.m - m0);
  const __amdgpu_buffer_rsrc_t xbuf = byte_buffer(
      a.x + uint64_t(m0) * a.ldx, uint32_t(((rows - 1) * a.ldx + a.k) * 2));
  // MFMA lane 16 h + r takes A row r (row m of class c) and the 8 k of
  // k-slot h of its block: 16 bytes at byte 64 c + 16 h of the register's
  // P-block span, so an A row's four k-slots are one contiguous 64-byte run.
  // The load itself assigns that run to the lane quad 4 r .. 4 r + 3 (lane
  // 4 r + h reads k-slot h), which the texture path serves as one 64-byte
  // access per quad instead of four (a quad of MFMA lanes spans four rows),
  // and a lane permute (xperm) then hands each lane its MFMA operand.
  // Measured on MI355X (TCP_TOTAL_CACHE_ACCESSES, AQ4 M=8 14336->4096):
  // 64 accesses per activation load in MFMA order, against 16 for a
  // contiguous kilobyte.
  uint32_t xoff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint32_t r = lane / 4, h = lane % 4;
    const uint32_t m = mt * 16 + r % RP;
    const uint32_t c = r / RP;
    xoff[mt] = m < rows ? uint32_t((m * a.ldx + 8 * h) * 2 + 64 * c)
                        : 0x80000000u;
  }
  // Source lane of MFMA lane 16 h + r: 4 r + h (byte address for bpermute).
  const int xsrc = int(((lane % 16) * 4 + lane / 16) * 4);
  auto xperm = [&](bf16x8 v) {
    u32x4 u = __builtin_bit_cast(u32x4, v);
    u32x4 o;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      o[d] = uint32_t(__builtin_amdgcn_ds_bpermute(xsrc, int(u[d])));
    }
    return __builtin_bit_cast(bf16x8, o);
  };
  // Class of this lane's accumulator rows 4 (l / 16) .. + 3.
  const uint32_t lcls = (lane / 16) * 4 / RP;
  const uint32_t wlane = lane * 16, zlane = (lane % 16) * 4;
  const bf16x8 ones = __builtin_bit_cast(
      bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
  const uint32_t nmask = opaque_u32(0x000f000fu);
  const uint32_t nmagic = opaque_u32(0x43004300u);

  struct Batch {
    u32x4 w[B][S];
    uint32_t sz[B][S];
    bf16x8 x[B][MT][XR];
  };
  uint32_t lg = 0, lu = ub;
  auto issue = [&](Batch &bt) {
    const uint32_t xpast = lg < nG ? 0u : 0x80000000u;
#pragma unroll
    for (int i = 0; i < B; ++i) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int t = 0; t < XR; ++t) {
          bt.x[i][mt][t] = __builtin_bit_cast(
              bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                          xbuf, xoff[mt],
                          ((lu + i) * 256 + t * P * 64) | xpast, 0));
        }
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const uint32_t item = (lg * S + s) * groups + lu + i;
        bt.w[i][s] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(wbuf, wlane,
                                                         item * 1024, kNt));
        bt.sz[i][s] =
            __builtin_amdgcn_raw_buffer_load_b32(zbuf, zlane, item * 64, 0);
      }
    }
    lu += B;
    if (lu == ue) {
      lu = ub;
      ++lg;
    }
  };

  Batch ring[DEPTH];
#pragma unroll
  for (int r = 0; r + 1 < DEPTH; ++r) {
    issue(ring[r]);
    // Keep the batches in ring order: the steady-state waits assume that
    // batch r's loads are all older than batch r + 1's.
    __builtin_amdgcn_sched_barrier(0);
  }
  f32x4 acc[S][MT];
  auto zero_acc = [&]() {
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[s][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  zero_acc();
  uint32_t cgp = 0, cu = ub;
  auto consume = [&](const Batch &bt) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      bf16x8 xv[MT][XR];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int t = 0; t < XR; ++t) {
          xv[mt][t] = xperm(bt.x[i][mt][t]);
        }
      }
      f32x4 xsum[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        xsum[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < XR; ++t) {
          xsum[mt] = mfma_bf16(xv[mt][t], ones, xsum[mt]);
        }
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        f32x4 p[P][MT];
#pragma unroll
        for (int c = 0; c < P; ++c) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            p[c][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8 bj = nib8_to_bf16_off128(bt.w[i][s][j], nmask, nmagic);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            p[j % P][mt] = mfma_bf16(xv[mt][j / P], bj, p[j % P][mt]);
          }
        }
        const float sf = f16_to_f32(uint16_t(bt.sz[i][s] & 0xffffu));
        const float zoff = 128.0f + f16_to_f32(uint16_t(bt.sz[i][s] >> 16));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          f32x4 q = p[0][mt];
#pragma unroll
          for (int c = 1; c < P; ++c) {
            q = lcls == uint32_t(c) ? p[c][mt] : q;
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc[s][mt][r] += sf * (q[r] - zoff * xsum[mt][r]);
          }
        }
      }
    }
    cu += B;
    if (cu == ue) {  // stripe group done: reduce across waves, store, reset
      float *rb = red[cgp & 1];
#pragma unroll
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            rb[(((wave * S + s) * MT + mt) * 4 + r) * kWave + lane] = acc[s][mt][r];
          }
        }
      }
      lds_barrier();
      const uint32_t Tg = T0 + cgp * S;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        // Output row mrow of the m-tile is the sum of accumulator row
        // c RP + mrow over the classes c.
        for (uint32_t o = threadIdx.x; o < MT * RP * 16; o += WAVES * kWave) {
          const uint32_t mt = o / (RP * 16), mrow = (o % (RP * 16)) / 16;
          const uint32_t ncol = o % 16;
          float v = 0.0f;
#pragma unroll
          for (int c = 0; c < P; ++c) {
            const uint32_t arow = c * RP + mrow;
            const uint32_t src = ncol + 16 * (arow / 4), r = arow % 4;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
              v += rb[(((w * S + s) * MT + mt) * 4 + r) * kWave + src];
            }
          }
          const uint32_t m = m0 + mt * 16 + mrow, n = (Tg + s) * 16 + ncol;
          if constexpr (SK) {
            // A ragged last group's missing stripes have no slot (slot
            // stripes would alias the next K part's stripe 0).
            if (Tg + s < stripes) {
              sk_put(pbuf,
                     ((uint64_t(kp) * stripes + Tg + s) * (MT * 16) + mt * 16 + mrow) * 16 +
                         ncol,
                     v);
            }
          } else {
            store_out<EPI>(a.y, a.ldy, a.y_f32, a.epi, a.n, m, n, a.alpha * v,
                    m < a.m);
          }
        }
      }
      if constexpr (SK) {
        if (sk_arrive(a.cnt + G0 + cgp, ks, &sk_flag)) {
#pragma unroll
          for (int s = 0; s < S; ++s) {
            if (Tg + s >= stripes) {
              break;
            }
            for (uint32_t o = threadIdx.x; o < MT * RP * 16; o += WAVES * kWave) {
              const uint32_t mt = o / (RP * 16), mrow = (o % (RP * 16)) / 16;
              const uint32_t ncol = o % 16;
              float v = 0.0f;
              for (uint32_t k = 0; k < ks; ++k) {
                v += sk_get(pbuf, ((uint64_t(k) * stripes + Tg + s) * (MT * 16) +
                                     mt * 16 + mrow) * 16 + ncol);
              }
              const uint32_t m = m0 + mt * 16 + mrow, n = (Tg + s) * 16 + ncol;
              store_out<EPI>(a.y, a.ldy, a.y_f32, a.epi, a.n, m, n, a.alpha * v,
                    m < a.m);
            }
          }
        }
      }
      zero_acc();
      cu = ub;
      ++cgp;
    }
  };

  for (uint32_t t = 0; t < NB; t += DEPTH) {
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) {
      issue(ring[(r + DEPTH - 1) % DEPTH]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + r < NB) {
        consume(ring[r]);
      }
    }
  }
}

// Waves per workgroup (they split K).  Measured on MI355X: FP8 streams best
// with 8 waves per stripe at every Llama shape; AQ4 (half the bytes per
// stripe) with 4 once the grid has enough stripes to fill the chip.
int pick_waves(bool aq4, uint64_t stripes, uint64_t mblocks, uint32_t units) {
  static const int forced = [] {
    const char *e = tuning_env("ULLM_GEMV_WAVES");
    return e ? std::atoi(e) : 0;
  }();
  if (forced == 2 || forced == 4 || forced == 8 || forced == 16) {
    return forced;
  }
  int waves = aq4 && stripes * mblocks >= 512 ? 4 : 8;
  while (waves > 2 && uint32_t(waves) > units) {
    waves /= 2;
  }
  return waves;
}

// Tuning override: ULLM_GEMV_LDS=0 disables the LDS-staged variant.
bool lds_allowed() {
  static const bool ok = [] {
    const char *e = tuning_env("ULLM_GEMV_LDS");
    return !(e && e[0] == '0');
  }();
  return ok;
}

// Tuning override: ULLM_GEMV_LDS_KB caps the staged activation block.
uint32_t lds_cap(bool aq4) {
  static const uint32_t forced = [] {
    const char *e = tuning_env("ULLM_GEMV_LDS_KB");
    return e ? uint32_t(std::atoi(e)) * 1024u : 0u;
  }();
  const uint32_t cap = aq4 ? kXLdsBytesAq4 : kXLdsBytes;
  return forced != 0 && forced <= kXLdsBytes ? forced : cap;
}

// Launch with `bytes` of dynamic LDS, raising the kernel's limit past the
// 64 KiB default once per kernel.
template <typename Kernel>
hipError_t launch_lds(Kernel kernel, dim3 grid, dim3 block, uint32_t bytes,
                      hipStream_t s, const GemvArgs &a) {
  if (bytes > 64 * 1024) {
    // Raise the kernel's dynamic-LDS limit to what this launch needs (the
    // limit plus the kernel's static LDS may not exceed the CU's 160 KiB).
    static std::mutex mu;
    static std::unordered_map<const void *, uint32_t> raised;
    std::lock_guard<std::mutex> lock(mu);
    const void *key = reinterpret_cast<const void *>(kernel);
    auto it = raised.find(key);
    if (it == raised.end() || it->second < bytes) {
      const hipError_t e = hipFuncSetAttribute(
          key, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
      if (e != hipSuccess) {
        return e;
      }
      raised[key] = bytes;
    }
  }
  hipLaunchKernelGGL(kernel, grid, block, bytes, s, a);
  return hipGetLastError();
}

// Activation rows plus the zero row, plus the AQ4 group sums.
uint32_t lds_bytes(const GemvArgs &a, bool aq4) {
  const uint32_t rows = min(a.m, 32u);
  return (rows + 1) * a.k * 2 + (aq4 ? rows * (a.k / 128) * 4 : 0);
}

// The single-stripe kernels stage the activation block in LDS when it fits.
bool single_uses_lds(const GemvArgs &a, bool vec, bool aq4) {
  return vec && lds_allowed() && lds_bytes(a, aq4) <= lds_cap(aq4);
}

template <int MT, int WAVES, int EPI>
hipError_t launch_fp8_t(const GemvArgs &a, bool vec, hipStream_t s) {
  const dim3 grid(a.n16 / 16, (a.m + 31) / 32);
  if (single_uses_lds(a, vec, false)) {
    if (a.units % (WAVES * kFp8LdsBatch) == 0) {
      return launch_lds(fp8_gemv_lds_kernel<MT, WAVES, kFp8LdsBatch, true, EPI>,
                        grid, dim3(WAVES * kWave), lds_bytes(a, false), s, a);
    }
    return launch_lds(fp8_gemv_lds_kernel<MT, WAVES, kFp8LdsBatch, false, EPI>,
                      grid, dim3(WAVES * kWave), lds_bytes(a, false), s, a);
  } else if (vec) {
    hipLaunchKernelGGL((fp8_gemv_kernel<MT, WAVES, true, EPI>), grid,
                       dim3(WAVES * kWave), 0, s, a);
  } else {
    hipLaunchKernelGGL((fp8_gemv_kernel<MT, WAVES, false, EPI>), grid,
                       dim3(WAVES * kWave), 0, s, a);
  }
  return hipGetLastError();
}

int env_int(const char *name, int dflt) {
  const char *e = tuning_env(name);
  return e ? std::atoi(e) : dflt;
}

// Multi-stripe kernels: as many workgroups as the device holds at once (by
// the occupancy calculator: registers and LDS), each walking a run of
// consecutive stripes.
template <typename Kernel>
uint32_t resident_blocks(Kernel kernel, uint32_t threads, uint32_t lds) {
  static std::mutex mu;
  static std::unordered_map<uint64_t, uint32_t> cache;
  int dev = 0;
  (void)hipGetDevice(&dev);
  const uint64_t key = (uint64_t(reinterpret_cast<uintptr_t>(
                            reinterpret_cast<const void *>(kernel))) << 8) ^
                       (uint64_t(lds) << 20) ^ uint64_t(dev);
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) {
    return it->second;
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, reinterpret_cast<const void *>(kernel), int(threads),
          size_t(lds)) != hipSuccess || per_cu < 1) {
    per_cu = 1;
  }
  const uint32_t n = device_cu_count() * uint32_t(per_cu);
  cache[key] = n;
  return n;
}

// Multi-stripe kernel configurations (waves, units per batch, ring depth),
// chosen by measurement on MI355X; overridable at build time for tuning.
#ifndef ULLM_AQ4_MS_CFG
#define ULLM_AQ4_MS_CFG 8, 2, 2, 8
#endif
#ifndef ULLM_FP8_MS_CFG
#define ULLM_FP8_MS_CFG 8, 4, 2, 8
#endif
struct MsCfg {
  int waves, batch, depth, ks;  // ks: waves splitting one stripe's K
};
constexpr MsCfg kAq4Ms{ULLM_AQ4_MS_CFG};
// AQ4 at M <= 2 with 6 (M = 1) or 3 (M = 2) to 16 stripes per CU: 4 waves,
// each owning whole stripes (no cross-wave reduction), 4 groups per batch.
// Measured on MI355X (K = 4096): M=1 4096->28672 12.7-12.8 against 14.6 us,
// M=2 4096->14336 8.2 against 9.1 us; M=1 4096->14336 (3.5 stripes per CU)
// level (7.65 against 7.68 us, kept on the default); behind at 1.5 and 31
// stripes per CU (M=1 4096->6144 6.8 against 5.0 us, 4096->128256 51-53
// against 46-48 us).
constexpr MsCfg kAq4MsWhole{4, 4, 2, 1};
constexpr MsCfg kFp8Ms{ULLM_FP8_MS_CFG};

// Register-staged kernel configurations by grid size (measured on MI355X,
// K = 4096 unless noted, against the kernel the launch used before):
//   wide   (>= 4096 stripes): 8 waves, groups of 4 stripes;
//          AQ4 M=8 4096->128256 54.5 against 59.7 us;
//   large  (>= 1024 stripes): 4 waves, groups of 4; AQ4 M=32 4096->28672
//          25.6 against 56.7 us, M=8 15.6 against 18.2 us; FP8 M=32 29.1
//          against 58.3 us;
//   medium (>= 384 stripes): 4 waves, groups of 2; AQ4 M=32 4096->6144 11.2
//          against 17.9 us, M=8 6.4 against 7.9 us;
//   deep K (< 384 stripes, K >= 8192): 16 waves, single stripes; AQ4 M=8
//          14336->4096 13.0 against 14.3 us (11.7 with rows packed);
//   small  (< 384 stripes, M <= 8, rows packed): 8 waves, single stripes;
//          AQ4 M=8 4096->4096 4.9 against 5.3 us;
//   small, wide rows (< 384 stripes, AQ4 16 <= M <= 32; FP8 see below):
//          4 waves, single stripes; 4096->4096 AQ4 M=16 6.16 against 6.35,
//          M=32 9.66 against 10.29, FP8 M=24 8.97 against 9.34, M=32 10.16
//          against 10.6 us (at FP8 M=17 and AQ4 M=9 the kernels used before
//          stay ahead: 7.3 against 8.2, 5.2 against 5.6 us).
//   FP8 medium and small, wide rows: 8 waves (groups of 2 and single
//          stripes); M=32 4096->6144 10.4 against 10.8 us, 4096->4096 M=24
//          8.6 against 9.5, M=32 9.2 against 9.6, M=23 8.6 against 9.1
//          and M=16 6.4 against 6.7 us (the LDS-staged kernel); at M = 17
//          and 18 the per-stripe kernel stays ahead (7.2 against 8.4, 8.3
//          against 8.5 us), level at M = 20 (AQ4 keeps 4 waves: its M=32
//          measured 9.3 against 8.8 and 7.6 against 7.1 us with 8);
//   deep K, FP8: 8 waves, single stripes, ring depth 3; FP8 M=8
//          14336->4096 12.8 against 14.0 us (median of 5; AQ4 keeps 16
//          waves: its M=8 measured level to slower with 8);
//   medium, AQ4 M <= 8: 4 waves, single stripes (rows then packed two or
//          four classes deep); 4096->6144 M=8 5.9 against 6.4 us, M=4 5.9
//          against 6.4 us, 4096->8192 M=8 6.3-6.6 against 6.9 us (at M=16
//          and 32 the groups of 2 stay ahead: 6.5 against 7.9, 8.8 against
//          11.4 us);
//   seven per CU (exactly 7 stripes per CU; AQ4 at every M, FP8 at M >= 16):
//          4 waves, groups of 7, one group per CU instead of 1.75 groups
//          of 4, so each CU reads the activation block once; 4096->28672
//          (1792 stripes on
//          256 CUs) AQ4 M=8 14.8-15.3 against 15.7-15.8 us, M=16 15.3-16.1
//          against 16.1-16.4, M=20 18.6 against 19.8, M=24 19.0 against
//          20.3, M=32 22.5 against 23.8 us; FP8 M=20 25.0 against 28.5,
//          M=24 25.1 against 29.3, M=32 26.9 against 31.3 us, M=16 22.0
//          against 22.5 us for the LDS-staged multi-stripe kernel (which
//          keeps M <= 12: level at 12, ahead at 8 and 9, 21.6 against 22.1
//          and 21.4 against 21.8 us).
// Each is {waves, units per batch, ring depth, stripes per group}.
struct RsCfg {
  int waves, batch, depth, s;
};
#ifndef ULLM_RS_WIDE
#define ULLM_RS_WIDE 8, 1, 2, 4
#endif
#ifndef ULLM_RS_LARGE
#define ULLM_RS_LARGE 4, 1, 2, 4
#endif
#ifndef ULLM_RS_MEDIUM
#define ULLM_RS_MEDIUM 4, 1, 2, 2
#endif
#ifndef ULLM_RS_DEEPK
#define ULLM_RS_DEEPK 16, 1, 2, 1
#endif
#ifndef ULLM_RS_SMALL
#define ULLM_RS_SMALL 8, 1, 2, 1
#endif
#ifndef ULLM_RS_SMALL_WIDE
#define ULLM_RS_SMALL_WIDE 4, 1, 2, 1
#endif
constexpr RsCfg kRsWide{ULLM_RS_WIDE};
constexpr RsCfg kRsLarge{ULLM_RS_LARGE};
#ifndef ULLM_RS_SEVEN
#define ULLM_RS_SEVEN 4, 1, 2, 7
#endif
constexpr RsCfg kRsSeven{ULLM_RS_SEVEN};
constexpr RsCfg kRsMediumPacked{4, 1, 2, 1};
constexpr RsCfg kRsDeepKFp8{8, 1, 3, 1};
constexpr RsCfg kRsMediumFp8{8, 1, 2, 2};
constexpr RsCfg kRsSmallWideFp8{8, 1, 2, 1};
constexpr RsCfg kRsMedium{ULLM_RS_MEDIUM};
constexpr RsCfg kRsDeepK{ULLM_RS_DEEPK};
constexpr RsCfg kRsSmall{ULLM_RS_SMALL};
constexpr RsCfg kRsSmallWide{ULLM_RS_SMALL_WIDE};

// Whether the multi-stripe kernel takes this launch.  It stages the
// activation block once per workgroup and amortises it over a run of
// stripes.  Measured on MI355X (AQ4, K = 4096, 8 waves, batches of 2
// groups): M=1 4096->14336 8.2 against 8.6 us for the single-stripe kernel,
// M=8 4096->28672 15.9 against 23.0 us, M=8 4096->128256 51.3 against 89.0
// us; but at M >= 4 a run of under 3 stripes per workgroup (4096->6144 at
// M=8) loses to the register kernel, which reads only its share of x.
// ULLM_GEMV_MS=0/1 overrides the choice.
bool use_ms(const GemvArgs &a, bool vec, int mt, bool aq4) {
  static const int forced = env_int("ULLM_GEMV_MS", -1);
  const MsCfg c = aq4 ? kAq4Ms : kFp8Ms;
  if (!vec || !lds_allowed() || forced == 0) {
    return false;
  }
  const uint32_t lds = ms_lds_bytes(a);
  const uint32_t stripes = a.n16 / 16;
  // Dynamic (activation block) plus static (two reduction buffers) LDS must
  // fit the CU's 160 KiB; a run's weights must stay below 2 GiB (32-bit
  // buffer offsets; checked for the whole matrix, the longest possible run).
  if (lds > kXLdsBytes || lds + 2u * c.waves * mt * 1024u > 160u * 1024u ||
      a.units % uint32_t(c.ks * c.batch) != 0 ||
      uint64_t(stripes) * a.units * 1024u >= (uint64_t(1) << 31)) {
    return false;
  }
  // AQ4 takes this kernel only with its activation rows packed four classes
  // deep, so at M <= 4.
  static const int cap = env_int("ULLM_GEMV_PACK", 4);
  if (aq4 && (a.m > 4 || cap < 4)) {
    return false;
  }
  if (forced == 1) {
    return true;
  }
  // FP8 (measured, 8 waves, batches of 4 units): M=8 4096->28672 20.6
  // against 25.1 us, M=16 21.9 against 39.4 us, M=8 4096->6144 7.1 against
  // 7.9 us; at M = 1..4 the single-stripe kernel is level or ahead on the
  // larger shapes (M=1 4096->28672 20.2 against 21.5 us).
  if (!aq4) {
    // ... and at M < 8 on grids of at most one stripe per CU (4096 -> 4096
    // M=1: 4.79 against 5.03 us).
    // ... except at M >= 16 on small grids (< 384 stripes), where the
    // register-staged single-stripe tier of 8 waves is ahead (4096 -> 4096
    // M=16 6.46 against 6.66 us).
    // ... and at M >= 16 on grids of exactly 7 stripes per CU, where one
    // register-staged group of 7 per CU reads the activations once per CU.
    return (a.m >= 8 || stripes <= device_cu_count()) && !(a.m >= 16 && stripes < 384) &&
           !(a.m >= 16 && stripes == 7 * device_cu_count());
  }
  // AQ4: M <= 2, or runs of 3+ stripes, taking two resident workgroups per
  // CU when the activation block leaves room for two.  (At M = 4 the
  // register-staged kernel, planned first, takes every launch whose
  // activation block lies within 2 GiB.)
  const uint32_t per_cu = lds + 16u * 1024u <= 80u * 1024u ? 2u : 1u;
  return a.m <= 2 || stripes >= 3 * device_cu_count() * per_cu;
}

template <typename Kernel>
hipError_t launch_ms(Kernel kernel, GemvArgs a, int waves, uint32_t lds,
                     hipStream_t s, uint32_t subgroups = 1) {
  const uint32_t stripes = a.n16 / 16;
  const uint32_t target = resident_blocks(kernel, waves * kWave, lds);
  static const int forced = env_int("ULLM_GEMV_SPW", 0);
  // Runs are whole multiples of the sub-group count, so no sub-group idles.
  const uint32_t spw = forced > 0 ? uint32_t(forced) : (stripes + target - 1) / target;
  a.spw = (spw + subgroups - 1) / subgroups * subgroups;
  const dim3 grid((stripes + a.spw - 1) / a.spw, (a.m + 31) / 32);
  return launch_lds(kernel, grid, dim3(waves * kWave), lds, s, a);
}

// AQ4 multi-stripe launches at M <= 2 with 6 (M = 1) or 3 (M = 2) to 16
// stripes per CU take the whole-stripe configuration.
bool aq4_ms_whole(const GemvArgs &a) {
  const uint32_t stripes = a.n16 / 16, cus = device_cu_count();
  return a.m <= 2 && stripes >= (a.m == 1 ? 6 : 3) * cus && stripes < 16 * cus &&
         a.units % uint32_t(kAq4MsWhole.batch) == 0;
}

template <int NR, int EPI>
hipError_t launch_aq4_ms(const GemvArgs &a, hipStream_t s) {
  if (aq4_ms_whole(a)) {
    constexpr MsCfg c = kAq4MsWhole;
    return launch_ms(aq4_gemv_ms_kernel<c.waves, c.ks, c.batch, c.depth, NR, EPI>,
                     a, c.waves, ms_lds_bytes(a), s, c.waves / c.ks);
  }
  return launch_ms(
      aq4_gemv_ms_kernel<kAq4Ms.waves, kAq4Ms.ks, kAq4Ms.batch, kAq4Ms.depth, NR, EPI>,
      a, kAq4Ms.waves, ms_lds_bytes(a), s, kAq4Ms.waves / kAq4Ms.ks);
}

template <int MT, int EPI>
hipError_t launch_fp8_ms(const GemvArgs &a, hipStream_t s) {
  return launch_ms(
      fp8_gemv_ms_kernel<MT, kFp8Ms.waves, kFp8Ms.batch, kFp8Ms.depth, EPI>, a,
      kFp8Ms.waves, ms_lds_bytes(a), s);
}

// Configuration of the register-staged kernel for this launch, or nullptr:
// it needs aligned activations, whole batches per wave, 32-bit buffer
// offsets for the weights and the activation block, and pays from M = 4 on
// (below, the LDS-staged kernels stay ahead).  ULLM_GEMV_RS=0 disables it,
// ULLM_GEMV_RS=1 forces it at any M.
const RsCfg *plan_rs(const GemvArgs &a, bool vec, bool aq4) {
  static const int forced = env_int("ULLM_GEMV_RS", -1);
  const uint32_t rows = min(a.m, 32u);
  const uint32_t stripes = a.n16 / 16;
  if (forced == 0 || !vec || (a.m < 4 && forced != 1) ||
      uint64_t(stripes) * a.units * 1024u >= (uint64_t(1) << 31) ||
      (uint64_t(rows - 1) * a.ldx + a.k) * 2 >= (uint64_t(1) << 31)) {
    return nullptr;
  }
  const uint32_t cus = device_cu_count();
  const RsCfg *c = (aq4 || a.m >= 16) && stripes == 7 * cus ? &kRsSeven
                   : stripes >= 4096   ? &kRsWide
                   : stripes >= 1024 ? &kRsLarge
                   : stripes >= 384  ? (!aq4 ? &kRsMediumFp8
                                        : a.m <= 8 ? &kRsMediumPacked : &kRsMedium)
                   : a.k >= 8192     ? (aq4 ? &kRsDeepK : &kRsDeepKFp8)
                   : a.m <= 8        ? &kRsSmall
                   : aq4 && a.m >= 16 && a.m <= 32                   ? &kRsSmallWide
                   : !aq4 && (a.m == 16 || a.m > 20) && a.m <= 32     ? &kRsSmallWideFp8
                                     : nullptr;
  if (c == nullptr && forced == 1) {
    c = &kRsMedium;
  }
  if (c == nullptr || a.units % uint32_t(c->waves * c->batch) != 0) {
    return nullptr;
  }
  return c;
}

template <typename Kernel>
hipError_t launch_rs(Kernel kernel, const RsCfg &C, GemvArgs a,
                     hipStream_t s) {
  const uint32_t groups = (a.n16 / 16 + C.s - 1) / C.s;
  const uint32_t target = resident_blocks(kernel, C.waves * kWave, 0);
  static const int forced = env_int("ULLM_GEMV_SPW", 0);
  a.spw = forced > 0 ? uint32_t(forced) : (groups + target - 1) / target;
  const dim3 grid((groups + a.spw - 1) / a.spw, (a.m + 31) / 32);
  hipLaunchKernelGGL(kernel, grid, dim3(C.waves * kWave), 0, s, a);
  return hipGetLastError();
}

#define ULLM_RS_KERNEL(K, MT, C, P) K<MT, C.waves, C.s, C.batch, C.depth, P, EPI, false>
// The (configuration, m-tiles, row classes) combinations plan_rs and
// rs_pack can select: rows are packed only in single-stripe groups, and the
// tiers limited to M <= 16 never run two m-tiles.  Only these are compiled;
// any other combination reports an invalid launch.
constexpr bool rs_reachable(const RsCfg &c, int mt, int p) {
  return (p == 1 || c.s == 1) &&
         (mt == 1 || !(&c == &kRsMediumPacked || &c == &kRsSmall));
}
#define ULLM_RS_CASE(K, C)                                                  \
  if (c == &C) {                                                            \
    if constexpr (rs_reachable(C, MT, P)) {                                 \
      return launch_rs(ULLM_RS_KERNEL(K, MT, C, P), *c, a, s);              \
    } else {                                                                \
      return hipErrorInvalidValue;                                          \
    }                                                                       \
  }
template <int MT, int P, int EPI>
hipError_t launch_fp8_rs(const GemvArgs &a, const RsCfg *c, hipStream_t s) {
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsWide)
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsSeven)
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsLarge)
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsMedium)
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsDeepK)
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsDeepKFp8)
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsMediumFp8)
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsSmallWideFp8)
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsSmallWide)
  ULLM_RS_CASE(fp8_gemv_rs_kernel, kRsSmall)
  return hipErrorInvalidValue;
}

template <int MT, int P, int EPI>
hipError_t launch_aq4_rs(const GemvArgs &a, const RsCfg *c, hipStream_t s) {
  ULLM_RS_CASE(aq4_gemv_rs_kernel, kRsWide)
  ULLM_RS_CASE(aq4_gemv_rs_kernel, kRsLarge)
  ULLM_RS_CASE(aq4_gemv_rs_kernel, kRsSeven)
  ULLM_RS_CASE(aq4_gemv_rs_kernel, kRsMediumPacked)
  ULLM_RS_CASE(aq4_gemv_rs_kernel, kRsMedium)
  ULLM_RS_CASE(aq4_gemv_rs_kernel, kRsDeepK)
  ULLM_RS_CASE(aq4_gemv_rs_kernel, kRsSmallWide)
  ULLM_RS_CASE(aq4_gemv_rs_kernel, kRsSmall)
  return hipErrorInvalidValue;
}

// Split-K configurations: groups of adjacent stripes (shared activation
// loads), K split over ksplit workgroups per group.  Measured on MI355X at
// N = 4096, K = 14336 (medians of 3) against 4 waves in groups of 4: AQ4 in
// groups of 2, M=16 13.3 against 15.1 us, M=32 16.4 against 21.0 us; FP8
// with 8 waves, M=16 in groups of 2 15.9 against 17.5 us, M=24 and 32 in
// groups of 4 19.2 against 21.9 and 20.3 against 23.5 us.
constexpr RsCfg kRsSplitAq4{4, 1, 2, 2};
constexpr RsCfg kRsSplitFp8Narrow{8, 1, 2, 2};  // M <= 16
constexpr RsCfg kRsSplitFp8Wide{8, 1, 2, 4};    // 16 < M <= 32
constexpr uint32_t kSplitMinGroup = 2;           // smallest group of the three

// Counter words: one per stripe group.  The region has one size for every
// split launch (plan_split takes fewer than 384 stripes, so at most 192
// groups of the smallest group size): the counters of one launch then never
// overlap the partial sums an earlier launch with fewer stripes left in the
// same workspace, which would break the zero-on-entry invariant.
constexpr uint32_t kSplitMaxStripes = 384;
constexpr uint64_t kSplitCounterBytes = 1024;
static_assert((kSplitMaxStripes + kSplitMinGroup - 1) / kSplitMinGroup * 4 <= kSplitCounterBytes,
              "counter region holds one word per group");
uint64_t split_cnt_bytes(const GemvArgs &) { return kSplitCounterBytes; }

const RsCfg &split_cfg(const GemvArgs &a, bool aq4) {
  return aq4 ? kRsSplitAq4 : a.m <= 16 ? kRsSplitFp8Narrow : kRsSplitFp8Wide;
}

// K parts per stripe group for this launch (1 = no split): 9 <= M <= 32
// (one activation block), few stripes (< 384) and K >= 12288, with enough
// parts that groups x parts fill every CU, each part whole batches per wave.
// Measured on MI355X (N = 4096, K = 14336): FP8 M=16 17.3 against 18.7 us,
// M=32 23.7 against 29.9 us; AQ4 M=16 15.1 against 17.2 us, M=32 22.1
// against 29.8 us.  The finisher's round trips through memory (stores,
// counter, partial loads: ~5 us) cost more than the split saves at M <= 8
// (AQ4 M=8 14.3 against 11.8 us) and at K <= 8192.
// ULLM_GEMV_SPLIT=0 disables, =N forces N parts where they divide.
uint32_t plan_split(const GemvArgs &a, bool vec, bool aq4) {
  static const int forced = env_int("ULLM_GEMV_SPLIT", -1);
  const RsCfg &c = split_cfg(a, aq4);
  const uint32_t stripes = a.n16 / 16;
  const uint32_t k = a.units * (aq4 ? 128u : 64u);
  if (forced == 0 || !vec || a.m > 32 || stripes >= kSplitMaxStripes ||
      (forced < 0 && (k < 12288 || a.m <= 8)) ||
      uint64_t(stripes) * a.units * 1024u >= (uint64_t(1) << 31) ||
      (uint64_t(a.m - 1) * a.ldx + a.k) * 2 >= (uint64_t(1) << 31)) {
    return 1;
  }
  const uint32_t G = (stripes + c.s - 1) / c.s;
  uint32_t ks = forced > 1 ? uint32_t(forced) : (device_cu_count() + G - 1) / G;
  ks = std::min(ks, 16u);
  const uint32_t per = uint32_t(c.waves * c.batch);
  while (ks > 1 && a.units % (ks * per) != 0) {
    --ks;
  }
  return ks;
}


uint64_t split_bytes(const GemvArgs &a, uint32_t ks) {
  const uint64_t rows = a.m > 16 ? 32 : 16;
  return split_cnt_bytes(a) + uint64_t(ks) * a.n16 * rows * 4;
}

// One workgroup per (stripe group, K part).
template <typename Kernel>
hipError_t launch_split(Kernel kernel, const RsCfg &c, GemvArgs a, uint32_t ks,
                        hipStream_t s) {
  const uint32_t groups = (a.n16 / 16 + c.s - 1) / c.s;
  a.spw = 1;
  a.ksplit = ks;
  hipLaunchKernelGGL(kernel, dim3(groups * ks), dim3(c.waves * kWave), 0, s, a);
  return hipGetLastError();
}
#define ULLM_SPLIT_KERNEL(K, MT, C) K<MT, C.waves, C.s, C.batch, C.depth, 1, EPI, true>

// Row packing of the register-staged kernels: the largest P <= the cap
// whose classes (16 / P rows) hold M, for single-stripe groups only.  With
// groups of S >= 2 stripes the activation loads are already shared and the
// per-group class select costs more than the saved loads (MI355X, AQ4 M=4
// 4096->28672, groups of 4: 15.1 us unpacked, 15.2 at P = 2, 17.5 at P = 4;
// single stripes, M=4 14336->4096: 11.4, 9.8, 8.9 us).  ULLM_GEMV_PACK sets
// the cap (1 = no packing).
int rs_pack(const GemvArgs &a, const RsCfg *c, bool aq4) {
  static const int cap = env_int("ULLM_GEMV_PACK", 4);
  if (c->s != 1) {
    return 1;
  }
  if (cap >= 4 && aq4 && a.m <= 4) {
    return 4;
  }
  return cap >= 2 && a.m <= 8 ? 2 : 1;
}
#undef ULLM_RS_KERNEL
#undef ULLM_RS_CASE

template <int MT, int WAVES, int EPI>
hipError_t launch_aq4_t(const GemvArgs &a, bool vec, hipStream_t s) {
  const dim3 grid(a.n16 / 16, (a.m + 31) / 32);
  if (single_uses_lds(a, vec, true)) {
    if (a.units % (WAVES * kAq4LdsBatch) == 0) {
      return launch_lds(aq4_gemv_lds_kernel<MT, WAVES, kAq4LdsBatch, true, EPI>,
                        grid, dim3(WAVES * kWave), lds_bytes(a, true), s, a);
    }
    return launch_lds(aq4_gemv_lds_kernel<MT, WAVES, kAq4LdsBatch, false, EPI>,
                      grid, dim3(WAVES * kWave), lds_bytes(a, true), s, a);
  } else if (vec) {
    hipLaunchKernelGGL((aq4_gemv_kernel<MT, WAVES, true, EPI>), grid,
                       dim3(WAVES * kWave), 0, s, a);
  } else {
    hipLaunchKernelGGL((aq4_gemv_kernel<MT, WAVES, false, EPI>), grid,
                       dim3(WAVES * kWave), 0, s, a);
  }
  return hipGetLastError();
}

// Unconditional 16-byte activation reads need aligned rows and, for FP8, a
// K that fills every 64-wide unit (AQ4 K is always a multiple of 128).
bool x_vec_ok(const GemvArgs &a, uint32_t unit_k) {
  // The buffer descriptor of XRow<true> spans at most 32 rows; its byte
  // extent must stay below 2^31 so that the out-of-range offset is rejected.
  return (reinterpret_cast<uintptr_t>(a.x) % 16 == 0) && (a.ldx % 8 == 0) &&
         (a.k % unit_k == 0) &&
         (uint64_t(31) * a.ldx + a.k) * 2 < (uint64_t(1) << 31);
}

}  // namespace

// Compute units of the current device (cached per device).
uint32_t device_cu_count() {
  static std::mutex mu;
  static std::unordered_map<int, uint32_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    return 256;
  }
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) {
    return it->second;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
          hipSuccess || n <= 0) {
    n = 256;
  }
  cache[dev] = uint32_t(n);
  return uint32_t(n);
}

const char *tuning_env(const char *name) {
#ifdef ULLM_TUNING
  return std::getenv(name);
#else
  (void)name;
  return nullptr;
#endif
}

namespace {

// The launch plan of a decode call: which kernel family, and its shape.
// Both the launchers below and the forward plan take it from here.
struct Choice {
  GemvChoice info;
  const RsCfg *rs = nullptr;  // register-staged and split-K configuration
};

Choice choose_fp8(const GemvArgs &a, bool split_ok) {
  Choice c;
  const bool vec = x_vec_ok(a, 64);
  const bool two = a.m > 16;
  // FP8 keeps the LDS-staged kernel where the activation block fits (M=8
  // 4096->28672: 21.0 against 25.3 us register-staged); AQ4, whose per-byte
  // work is heavier, gains from the register-staged kernel there too.
  if (use_ms(a, vec, two ? 2 : 1, false)) {
    c.info.variant = ULLM_LINEAR_GEMV_MULTI_STRIPE;
    c.info.waves = kFp8Ms.waves;
    return c;
  }
  const uint32_t ks = split_ok && a.m >= 8 ? plan_split(a, vec, false) : 1;
  if (ks > 1) {
    c.rs = two ? &kRsSplitFp8Wide : &kRsSplitFp8Narrow;
    c.info.variant = ULLM_LINEAR_GEMV_SPLIT_K;
    c.info.ks = ks;
  } else if ((c.rs = a.m >= 8 ? plan_rs(a, vec, false) : nullptr)) {
    // At M < 8 the single-stripe LDS kernel below stays ahead for FP8.
    c.info.variant = ULLM_LINEAR_GEMV_REGISTER_STAGED;
    c.info.classes = two ? 1 : uint32_t(rs_pack(a, c.rs, false) == 2 ? 2 : 1);
  }
  if (c.rs != nullptr) {
    c.info.waves = c.rs->waves;
    c.info.stripes = c.rs->s;
    return c;
  }
  c.info.variant = single_uses_lds(a, vec, false) ? ULLM_LINEAR_GEMV_SINGLE_LDS
                                                  : ULLM_LINEAR_GEMV_SINGLE;
  c.info.waves = pick_waves(false, a.n16 / 16, (a.m + 31) / 32, a.units);
  return c;
}

Choice choose_aq4(const GemvArgs &a, bool split_ok) {
  Choice c;
  const bool vec = x_vec_ok(a, 128);
  const bool two = a.m > 16;
  const uint32_t ks = split_ok && a.m >= 4 ? plan_split(a, vec, true) : 1;
  if (ks > 1) {
    c.rs = &kRsSplitAq4;
    c.info.variant = ULLM_LINEAR_GEMV_SPLIT_K;
    c.info.ks = ks;
  } else if ((c.rs = plan_rs(a, vec, true))) {
    c.info.variant = ULLM_LINEAR_GEMV_REGISTER_STAGED;
    c.info.classes = two ? 1 : uint32_t(rs_pack(a, c.rs, true));
  }
  if (c.rs != nullptr) {
    c.info.waves = c.rs->waves;
    c.info.stripes = c.rs->s;
    return c;
  }
  if (use_ms(a, vec, 1, true)) {
    c.info.variant = ULLM_LINEAR_GEMV_MULTI_STRIPE;
    c.info.classes = 4;
    c.info.waves = aq4_ms_whole(a) ? kAq4MsWhole.waves : kAq4Ms.waves;
    return c;
  }
  c.info.variant = single_uses_lds(a, vec, true) ? ULLM_LINEAR_GEMV_SINGLE_LDS
                                                 : ULLM_LINEAR_GEMV_SINGLE;
  c.info.waves = pick_waves(true, a.n16 / 16, (a.m + 31) / 32, a.units);
  return c;
}

}  // namespace

template <int EPI>
hipError_t fp8_gemv_e(const GemvArgs &a, hipStream_t s) {
  const Choice c = choose_fp8(a, a.cnt != nullptr);
  const bool vec = x_vec_ok(a, 64);
  const bool two = a.m > 16;
  switch (c.info.variant) {
    case ULLM_LINEAR_GEMV_MULTI_STRIPE:
      return two ? launch_fp8_ms<2, EPI>(a, s) : launch_fp8_ms<1, EPI>(a, s);
    case ULLM_LINEAR_GEMV_SPLIT_K:
      return two ? launch_split(ULLM_SPLIT_KERNEL(fp8_gemv_rs_kernel, 2, kRsSplitFp8Wide),
                                kRsSplitFp8Wide, a, c.info.ks, s)
                 : launch_split(ULLM_SPLIT_KERNEL(fp8_gemv_rs_kernel, 1, kRsSplitFp8Narrow),
                                kRsSplitFp8Narrow, a, c.info.ks, s);
    case ULLM_LINEAR_GEMV_REGISTER_STAGED:
      if (two) {
        return launch_fp8_rs<2, 1, EPI>(a, c.rs, s);
      }
      return c.info.classes == 2 ? launch_fp8_rs<1, 2, EPI>(a, c.rs, s)
                                 : launch_fp8_rs<1, 1, EPI>(a, c.rs, s);
    default:
      break;
  }
  switch (c.info.waves * 2 + (two ? 1 : 0)) {
    case 4: return launch_fp8_t<1, 2, EPI>(a, vec, s);
    case 5: return launch_fp8_t<2, 2, EPI>(a, vec, s);
    case 8: return launch_fp8_t<1, 4, EPI>(a, vec, s);
    case 9: return launch_fp8_t<2, 4, EPI>(a, vec, s);
    case 16: return launch_fp8_t<1, 8, EPI>(a, vec, s);
    case 17: return launch_fp8_t<2, 8, EPI>(a, vec, s);
    case 32: return launch_fp8_t<1, 16, EPI>(a, vec, s);
    default: return launch_fp8_t<2, 16, EPI>(a, vec, s);
  }
}

template <int EPI>
hipError_t aq4_gemv_e(const GemvArgs &a, hipStream_t s) {
  const Choice c = choose_aq4(a, a.cnt != nullptr);
  const bool vec = x_vec_ok(a, 128);
  const bool two = a.m > 16;
  switch (c.info.variant) {
    case ULLM_LINEAR_GEMV_SPLIT_K:
      return two ? launch_split(ULLM_SPLIT_KERNEL(aq4_gemv_rs_kernel, 2, kRsSplitAq4),
                                kRsSplitAq4, a, c.info.ks, s)
                 : launch_split(ULLM_SPLIT_KERNEL(aq4_gemv_rs_kernel, 1, kRsSplitAq4),
                                kRsSplitAq4, a, c.info.ks, s);
    case ULLM_LINEAR_GEMV_REGISTER_STAGED:
      if (two) {
        return launch_aq4_rs<2, 1, EPI>(a, c.rs, s);
      }
      switch (c.info.classes) {
        case 4: return launch_aq4_rs<1, 4, EPI>(a, c.rs, s);
        case 2: return launch_aq4_rs<1, 2, EPI>(a, c.rs, s);
        default: return launch_aq4_rs<1, 1, EPI>(a, c.rs, s);
      }
    case ULLM_LINEAR_GEMV_MULTI_STRIPE:  // M <= 4, rows packed
      return a.m == 1 ? launch_aq4_ms<1, EPI>(a, s)
                      : a.m == 2 ? launch_aq4_ms<2, EPI>(a, s)
                                 : launch_aq4_ms<4, EPI>(a, s);
    default:
      break;
  }
  switch (c.info.waves * 2 + (two ? 1 : 0)) {
    case 4: return launch_aq4_t<1, 2, EPI>(a, vec, s);
    case 5: return launch_aq4_t<2, 2, EPI>(a, vec, s);
    case 8: return launch_aq4_t<1, 4, EPI>(a, vec, s);
    case 9: return launch_aq4_t<2, 4, EPI>(a, vec, s);
    case 16: return launch_aq4_t<1, 8, EPI>(a, vec, s);
    case 17: return launch_aq4_t<2, 8, EPI>(a, vec, s);
    case 32: return launch_aq4_t<1, 16, EPI>(a, vec, s);
    default: return launch_aq4_t<2, 16, EPI>(a, vec, s);
  }
}

// The epilogue kind is a template parameter of every kernel: dispatch once.
hipError_t launch_fp8_gemv(const GemvArgs &a, hipStream_t s) {
  switch (a.epi.kind) {
    case kEpiSiluMul: return fp8_gemv_e<kEpiSiluMul>(a, s);
    case kEpiResidual: return fp8_gemv_e<kEpiResidual>(a, s);
    default: return fp8_gemv_e<kEpiNone>(a, s);
  }
}

hipError_t launch_aq4_gemv(const GemvArgs &a, hipStream_t s) {
  switch (a.epi.kind) {
    case kEpiSiluMul: return aq4_gemv_e<kEpiSiluMul>(a, s);
    case kEpiResidual: return aq4_gemv_e<kEpiResidual>(a, s);
    default: return aq4_gemv_e<kEpiNone>(a, s);
  }
}

uint32_t gemv_split_parts(const GemvArgs &a, bool aq4) {
  return gemv_choice(a, aq4, true).ks;
}

GemvChoice gemv_choice(const GemvArgs &a, bool aq4, bool split_ok) {
  return (aq4 ? choose_aq4(a, split_ok) : choose_fp8(a, split_ok)).info;
}

uint64_t gemv_scratch_bytes(const GemvArgs &a, bool aq4) {
  const uint32_t ks = gemv_split_parts(a, aq4);
  return ks > 1 ? split_bytes(a, ks) : 0;
}

uint64_t gemv_scratch_part_offset(const GemvArgs &a) { return split_cnt_bytes(a); }

}  // namespace ullm
