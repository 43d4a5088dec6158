// gemm_step_probe.hip -- what one k-step of the prefill GEMM's main loop can
// cost on this part, measured without the GEMM around it.
//
// One round is one 256 x 256 x 128 k-step of a GEMM block on one CU: 64 KiB
// copied global -> LDS for the next stage (global_load_lds_dwordx4, 1 KiB per
// wave and copy), then every one of 8 waves reads TI A and TJ B operands from
// the current stage (two ds_read_b128 each) and runs TI x TJ
// v_mfma_scale_f32_16x16x128_f8f6f4, then waits for its copies and meets the
// others at a barrier.  256 workgroups (one per CU) run 2000 rounds over a
// 2 MiB source window that stays in L2.  The source is either constant bytes
// or hashed random E4M3 codes (no NaN), since switching activity sets the
// clock the part sustains.  s_memtime (shader clock) against the event time
// gives the clock.
//
// Build and run (gfx950):
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature \
//     -Xclang -packed-fp32-ops gemm_step_probe.hip -o gemm_step_probe
//   ./gemm_step_probe
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRounds = 2000;
constexpr int kGrid = 256;
constexpr unsigned kWindow = 2u << 20;  // bytes, a power of two

#define CHECK(x)                                                          \
  do {                                                                    \
    hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                               \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));        \
      std::exit(1);                                                       \
    }                                                                     \
  } while (0)

// Hashed bytes with the NaN code (S.1111.111) excluded.
__global__ void fill_random_e4m3(unsigned char *p, size_t n) {
  for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n;
       i += size_t(gridDim.x) * 256) {
    unsigned h = unsigned(i) * 2654435761u;
    h ^= h >> 13;
    h *= 0x5bd1e995u;
    h ^= h >> 15;
    p[i] = (unsigned char)((h & 0x7eu) | ((h >> 8) & 0x80u));
  }
}

__device__ __forceinline__ i32x8 operand(const char *q) {
  const u32x4 lo = *reinterpret_cast<const u32x4 *>(q);
  const u32x4 hi = *reinterpret_cast<const u32x4 *>(q + 1024);
  return i32x8{int(lo.x), int(lo.y), int(lo.z), int(lo.w),
               int(hi.x), int(hi.y), int(hi.z), int(hi.w)};
}

// COPY: issue the round's 64 KiB of copies; MF: read operands from LDS and
// run the MFMAs.
template <int TI, int TJ, bool COPY, bool MF>
__global__ __launch_bounds__(512) void step(const char *src, int rounds,
                                            float *out,
                                            unsigned long long *clk) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  unsigned off = (blockIdx.x * 64u * 1024u * 7u) & (kWindow - 1);
  f32x4 acc[TI * TJ];
#pragma unroll
  for (int j = 0; j < TI * TJ; ++j) {
    acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < rounds; ++it) {
    const int cur = it & 1, nxt = cur ^ 1;
    if (COPY) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const char *p = src + ((off + (c * 8 + wave) * 1024u) & (kWindow - 1)) +
                        lane * 16;
        __builtin_amdgcn_global_load_lds(
            (__attribute__((address_space(1))) void *)p,
            (__attribute__((address_space(3))) void *)(lds + (nxt * 64 + c * 8 + wave) * 1024),
            16, 0, 0);
      }
    }
    if (MF) {
      const char *st = lds + cur * 65536;
      i32x8 bf[TJ];
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        bf[j] = operand(st + 32768 + ((wave * TJ + j) * 2048 & 32767) + lane * 16);
      }
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const i32x8 af = operand(st + ((wave * TI + i) * 2048 & 32767) + lane * 16);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          acc[i * TJ + j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              af, bf[j], acc[i * TJ + j], 0, 0, 0, 0, 0, 0);
        }
      }
    }
    // Keep the MFMAs of this round ahead of its wait and barrier.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    off = (off + 64u * 1024u) & (kWindow - 1);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float t = 0.f;
#pragma unroll
  for (int j = 0; j < TI * TJ; ++j) {
    t += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  }
  out[blockIdx.x * 512 + threadIdx.x] = t;
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    clk[0] = t1 - t0;
  }
}

template <int TI, int TJ, bool COPY, bool MF>
void run(const char *name, const char *src, float *out,
         unsigned long long *clk) {
  auto kernel = step<TI, TJ, COPY, MF>;
  CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 131072));
  kernel<<<kGrid, 512, 131072>>>(src, 10, out, clk);
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  kernel<<<kGrid, 512, 131072>>>(src, kRounds, out, clk);
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  unsigned long long cycles = 0;
  CHECK(hipMemcpy(&cycles, clk, sizeof(cycles), hipMemcpyDeviceToHost));
  const double us = ms * 1e3 / kRounds;
  const double flop = MF ? 2.0 * 16 * 16 * 128 * TI * TJ * 8 * kGrid : 0.0;
  std::printf("%-40s %6.3f us/round %6.0f clk/round %5.0f MHz %6.0f TFLOP/s %5.1f TB/s copied\n",
              name, us, double(cycles) / kRounds, double(cycles) / (ms * 1e3),
              flop / (us * 1e-6) / 1e12,
              COPY ? 65536.0 * kGrid / (us * 1e-6) / 1e12 : 0.0);
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

}  // namespace

int main() {
  char *src = nullptr;
  float *out = nullptr;
  unsigned long long *clk = nullptr;
  CHECK(hipMalloc(&src, kWindow));
  CHECK(hipMalloc(&out, kGrid * 512 * sizeof(float)));
  CHECK(hipMalloc(&clk, sizeof(unsigned long long)));
  CHECK(hipMemset(src, 1, kWindow));
  std::printf("constant bytes:\n");
  run<8, 4, true, false>("copy only", src, out, clk);
  run<8, 4, true, true>("copy+lds+mfma, waves of 128x64", src, out, clk);
  run<4, 7, true, true>("copy+lds+mfma, waves of 64x112", src, out, clk);
  fill_random_e4m3<<<1024, 256>>>(reinterpret_cast<unsigned char *>(src), kWindow);
  CHECK(hipDeviceSynchronize());
  std::printf("random E4M3 codes:\n");
  run<8, 4, true, true>("copy+lds+mfma, waves of 128x64", src, out, clk);
  run<4, 7, true, true>("copy+lds+mfma, waves of 64x112", src, out, clk);
  CHECK(hipDeviceSynchronize());
  return 0;
}
