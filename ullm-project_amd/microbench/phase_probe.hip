// phase_probe.hip -- can one persistent kernel stream a decode step's
// projections faster than one launch per projection?
//
// A decode step streams the weights of its projections one after the other;
// each projection depends on the one before, so consecutive launches cannot
// overlap and every launch pays its own start (first bytes back from HBM)
// and drain.  A persistent grid that runs the projections as phases needs a
// grid-wide barrier between them instead, but the next phase's weight loads
// do not depend on the barrier and can be issued before waiting on it.
//
// Every phase here is a pure weight stream (1 KiB per wave and load, XOR
// reduced), with the byte counts of the batch-8 AQ4 stack's projections
// (qkv, o, gate_up, down) repeated for kLayers layers.  Ways to run it:
//   launches   one kernel per phase, captured in a HIP graph;
//   barrier    one persistent kernel (one workgroup per CU), each phase
//              starting its loads after the grid barrier;
//   prefetch   the same, with each wave's first 8 KiB of the next phase
//              issued between arriving at the barrier and waiting on it;
//   */nofence  both again with a relaxed add and no acquire fence (enough
//              here, where no phase reads what another wrote; a real step
//              would need the fences, or stores and loads that bypass L2).
// The barrier is a per-phase counter: one release add per workgroup after
// its phase, then a spin on an agent-scope load and an acquire fence.  The
// spin is bounded; a grid of one workgroup per CU is co-resident (checked
// against the occupancy API before launch), so the bound is never reached
// in a correct run, and reaching it is reported.
//
// Build and run (gfx950):
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature \
//     -Xclang -packed-fp32-ops phase_probe.hip -o phase_probe
//   ./phase_probe
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kLayers = 8;
constexpr int kChunk = 8;  // loads of 1 KiB in flight per wave and buffer
constexpr unsigned kSpinLimit = 1u << 22;

#define CHECK(x)                                                          \
  do {                                                                    \
    hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                               \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));        \
      std::exit(1);                                                       \
    }                                                                     \
  } while (0)

struct Phases {
  const u32x4 *base[64];
  unsigned tiles[64];  // 1 KiB tiles, a multiple of the wave count
  int count;
};

// Wave w of W streams tiles [w * n / W, (w + 1) * n / W) of a phase, in
// chunks of kChunk loads; the chunk's loads are clamped to the share.
struct Stream {
  const u32x4 *p;
  unsigned n, i;
};

__device__ __forceinline__ void issue(u32x4 (&v)[kChunk], const Stream &s,
                                      unsigned lane) {
#pragma unroll
  for (int c = 0; c < kChunk; ++c) {
    const unsigned t = min(s.i + c, s.n - 1);
    v[c] = __builtin_nontemporal_load(s.p + size_t(t) * 64 + lane);
  }
}

__device__ __forceinline__ unsigned fold(const u32x4 (&v)[kChunk]) {
  unsigned x = 0;
#pragma unroll
  for (int c = 0; c < kChunk; ++c) {
    x ^= v[c].x ^ v[c].y ^ v[c].z ^ v[c].w;
  }
  return x;
}

__device__ __forceinline__ Stream share(const Phases &ph, int p, unsigned gw,
                                        unsigned nw) {
  const unsigned n = ph.tiles[p] / nw;
  return Stream{ph.base[p] + size_t(gw) * n * 64, n, 0};
}

// Streams one phase, with its first chunk already issued into a.
__device__ __forceinline__ unsigned run_phase(Stream s, u32x4 (&a)[kChunk],
                                              u32x4 (&b)[kChunk],
                                              unsigned lane) {
  unsigned x = 0;
  for (s.i = kChunk; s.i < s.n; s.i += 2 * kChunk) {
    issue(b, s, lane);
    x ^= fold(a);
    if (s.i + kChunk < s.n) {
      Stream t = s;
      t.i += kChunk;
      issue(a, t, lane);
    }
    x ^= fold(b);
  }
  if ((s.n + kChunk - 1) / kChunk % 2 == 1) {
    x ^= fold(a);
  }
  return x;
}

// One launch per phase.
__global__ __launch_bounds__(kWaves * 64) void one_phase(Phases ph, int p,
                                                         unsigned *out) {
  const unsigned lane = threadIdx.x % 64;
  const unsigned gw = blockIdx.x * kWaves + threadIdx.x / 64;
  const Stream s = share(ph, p, gw, gridDim.x * kWaves);
  u32x4 a[kChunk], b[kChunk];
  issue(a, s, lane);
  const unsigned x = run_phase(s, a, b, lane);
  if (x == 0x9e3779b9u) {
    out[0] = x;
  }
}

// All phases in one grid.  PREFETCH: issue the next phase's first chunk
// between arriving and waiting.
template <bool PREFETCH, bool FENCE = true>
__global__ __launch_bounds__(kWaves * 64) void persistent(Phases ph,
                                                          unsigned *cnt,
                                                          unsigned *out) {
  const unsigned lane = threadIdx.x % 64;
  const unsigned nw = gridDim.x * kWaves;
  const unsigned gw = blockIdx.x * kWaves + threadIdx.x / 64;
  u32x4 a[kChunk], b[kChunk];
  unsigned x = 0;
  issue(a, share(ph, 0, gw, nw), lane);
  for (int p = 0; p < ph.count; ++p) {
    x ^= run_phase(share(ph, p, gw, nw), a, b, lane);
    if (p + 1 == ph.count) {
      break;
    }
    // Every wave of the workgroup is done with phase p (LDS-only barrier:
    // no wait on outstanding vector loads).
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    if (threadIdx.x == 0) {
      if (FENCE) {
        __hip_atomic_fetch_add(cnt + p, 1u, __ATOMIC_RELEASE,
                               __HIP_MEMORY_SCOPE_AGENT);
      } else {
        __hip_atomic_fetch_add(cnt + p, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (PREFETCH) {
      issue(a, share(ph, p + 1, gw, nw), lane);
    }
    if (threadIdx.x == 0) {
      unsigned spins = 0;
      while (__hip_atomic_load(cnt + p, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT) < gridDim.x &&
             ++spins < kSpinLimit) {
        __builtin_amdgcn_s_sleep(1);
      }
      if (spins >= kSpinLimit) {
        __hip_atomic_fetch_add(out + 1, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      }
      if (FENCE) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    if (!PREFETCH) {
      issue(a, share(ph, p + 1, gw, nw), lane);
    }
  }
  if (x == 0x9e3779b9u) {
    out[0] = x;
  }
}

__global__ void fill(unsigned *p, size_t n) {
  for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n;
       i += size_t(gridDim.x) * 256) {
    unsigned h = unsigned(i) * 2654435761u;
    h ^= h >> 15;
    p[i] = h;
  }
}

}  // namespace

int main() {
  int dev = 0, cus = 0, per_cu = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(
      &per_cu, reinterpret_cast<const void *>(persistent<true>), kWaves * 64, 0));
  if (per_cu < 1) {
    std::fprintf(stderr, "persistent kernel not resident\n");
    return 1;
  }
  const unsigned grid = unsigned(cus);
  const unsigned nw = grid * kWaves;
  // Projection bytes of one batch-8 AQ4 layer: qkv, o, gate_up, down.
  const double layer_mb[4] = {13.4, 8.9, 62.4, 31.2};
  Phases ph{};
  size_t total_tiles = 0;
  std::vector<unsigned> tiles;
  for (int l = 0; l < kLayers; ++l) {
    for (int j = 0; j < 4; ++j) {
      unsigned t = unsigned(layer_mb[j] * 1e6 / 1024.0);
      t = (t + nw * kChunk - 1) / (nw * kChunk) * (nw * kChunk);
      tiles.push_back(t);
      total_tiles += t;
    }
  }
  ph.count = int(tiles.size());
  unsigned *buf = nullptr, *cnt = nullptr, *out = nullptr;
  CHECK(hipMalloc(&buf, total_tiles * 1024));
  CHECK(hipMalloc(&cnt, 64 * sizeof(unsigned)));
  CHECK(hipMalloc(&out, 2 * sizeof(unsigned)));
  CHECK(hipMemset(out, 0, 2 * sizeof(unsigned)));
  fill<<<2048, 256>>>(buf, total_tiles * 256);
  size_t off = 0;
  for (int p = 0; p < ph.count; ++p) {
    ph.base[p] = reinterpret_cast<const u32x4 *>(buf) + off * 64;
    ph.tiles[p] = tiles[p];
    off += tiles[p];
  }
  const double bytes = double(total_tiles) * 1024;
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  auto report = [&](const char *name, float ms, int reps) {
    const double us = ms * 1e3 / reps;
    std::printf("%-17s %8.1f us per %d phases  %6.2f us/phase  %5.2f TB/s\n",
                name, us, ph.count, us / ph.count, bytes / (us * 1e-6) / 1e12);
  };
  const int reps = 20;
  // Launches, captured in a graph.
  hipGraph_t g;
  hipGraphExec_t ge;
  CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
  for (int p = 0; p < ph.count; ++p) {
    one_phase<<<grid, kWaves * 64, 0, st>>>(ph, p, out);
  }
  CHECK(hipStreamEndCapture(st, &g));
  CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  for (int round = 0; round < 2; ++round) {
    CHECK(hipGraphLaunch(ge, st));
    CHECK(hipEventRecord(e0, st));
    for (int r = 0; r < reps; ++r) {
      CHECK(hipGraphLaunch(ge, st));
    }
    CHECK(hipEventRecord(e1, st));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    report("launches", ms, reps);
    for (int mode = 0; mode < 4; ++mode) {
      auto k = mode == 0   ? persistent<false, true>
               : mode == 1 ? persistent<true, true>
               : mode == 2 ? persistent<false, false>
                           : persistent<true, false>;
      CHECK(hipMemsetAsync(cnt, 0, 64 * sizeof(unsigned), st));
      k<<<grid, kWaves * 64, 0, st>>>(ph, cnt, out);
      CHECK(hipEventRecord(e0, st));
      for (int r = 0; r < reps; ++r) {
        CHECK(hipMemsetAsync(cnt, 0, 64 * sizeof(unsigned), st));
        k<<<grid, kWaves * 64, 0, st>>>(ph, cnt, out);
      }
      CHECK(hipEventRecord(e1, st));
      CHECK(hipEventSynchronize(e1));
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      static const char *names[4] = {"barrier", "prefetch", "barrier/nofence", "prefetch/nofence"};
      report(names[mode], ms, reps);
    }
  }
  unsigned h[2];
  CHECK(hipMemcpy(h, out, sizeof(h), hipMemcpyDeviceToHost));
  std::printf("spin limit reached: %u times\n", h[1]);
  return 0;
}
