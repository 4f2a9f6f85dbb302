// hbm_probe.hip — streaming probes that measure what the HBM of one gfx950
// GPU sustains for a given mix of read and write streams, independent of the
// boundary kernels.  They give the ceilings the boundary kernels are judged
// against: one read stream, one write stream, a copy, in-place
// read-modify-write of one or more arrays (the AdamW pattern: p, m, v read and
// written back at the same index) and any mix of those, with the launch shape
// (threads per block, 16-byte vectors in flight per lane, lane layout, one
// tile per block or a persistent grid, non-temporal hints) as parameters.
//
// Every stream is an array of 16-byte vectors; array k of a launch is read
// (k < nread), written (k < nwrite), or both when rd[k] == wr[k].  A block
// takes tiles of threads*unroll vectors.  With the "lane" layout lane j of a
// tile owns `unroll` consecutive vectors (the boundary kernels' layout: 8
// fp32 elements = 2 vectors per lane); with the "wave" layout load u of lane j
// is vector u*threads + j, so each load instruction covers one contiguous
// 64-lane run.  Written values are the read values plus one (or a constant
// when nothing is read); read-only launches fold everything they load into a
// value that is stored only if it equals an improbable constant, so the
// loads stay and nothing is written.
//
// Not on the boundary path: bench.py's --hbm-ceilings mode loads this
// library (libms_hbm_probe.so) and nothing else does.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "minispeed_hbm_probe.h"

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kMaxThreads = 1024;

struct ProbeArgs {
  const u4* rd[MSP_MAX_ARRAYS];
  u4* wr[MSP_MAX_ARRAYS];
  int nread, nwrite;
  int64_t nvec;
  uint32_t* sink;
};

template <bool kNt>
__device__ inline u4 ld(const u4* p) {
  if constexpr (kNt) return __builtin_nontemporal_load(p);
  return *p;
}

template <bool kNt>
__device__ inline void st(u4* p, u4 x) {
  if constexpr (kNt)
    __builtin_nontemporal_store(x, p);
  else
    *p = x;
}

template <int U, bool kWave, bool kNtLoad, bool kNtStore>
__global__ __launch_bounds__(kMaxThreads) void k_probe(ProbeArgs a) {
  const int threads = blockDim.x;
  const int lane = threadIdx.x;
  const int64_t per_tile = static_cast<int64_t>(threads) * U;
  const int64_t ntiles = (a.nvec + per_tile - 1) / per_tile;
  u4 fold = {0u, 0u, 0u, 0u};
  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    int64_t idx[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      idx[u] = t * per_tile + (kWave ? static_cast<int64_t>(u) * threads + lane
                                     : static_cast<int64_t>(lane) * U + u);
    u4 x[MSP_MAX_ARRAYS][U];
#pragma unroll
    for (int k = 0; k < MSP_MAX_ARRAYS; ++k) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        x[k][u] = u4{1u, 2u, 3u, 4u};
        if (k < a.nread && idx[u] < a.nvec) x[k][u] = ld<kNtLoad>(a.rd[k] + idx[u]);
      }
    }
#pragma unroll
    for (int k = 0; k < MSP_MAX_ARRAYS; ++k) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (k < a.nwrite && idx[u] < a.nvec) st<kNtStore>(a.wr[k] + idx[u], x[k][u] + 1u);
        if (k < a.nread) fold ^= x[k][u];
      }
    }
  }
  if (a.nwrite == 0 && fold.x == 0x9e3779b9u && fold.y == 0x7f4a7c15u && fold.z == 0x85ebca6bu &&
      fold.w == 0xc2b2ae35u)
    a.sink[blockIdx.x & 1023] = fold.x ^ fold.y ^ fold.z ^ fold.w;
}

template <int U, bool kWave>
void launch_nt(const ProbeArgs& a, int grid, int threads, int nt_load, int nt_store, hipStream_t s) {
  if (nt_load && nt_store)
    hipLaunchKernelGGL((k_probe<U, kWave, true, true>), dim3(grid), dim3(threads), 0, s, a);
  else if (nt_load)
    hipLaunchKernelGGL((k_probe<U, kWave, true, false>), dim3(grid), dim3(threads), 0, s, a);
  else if (nt_store)
    hipLaunchKernelGGL((k_probe<U, kWave, false, true>), dim3(grid), dim3(threads), 0, s, a);
  else
    hipLaunchKernelGGL((k_probe<U, kWave, false, false>), dim3(grid), dim3(threads), 0, s, a);
}

template <int U>
void launch_u(const ProbeArgs& a, int grid, int threads, int wave, int nt_load, int nt_store,
              hipStream_t s) {
  if (wave)
    launch_nt<U, true>(a, grid, threads, nt_load, nt_store, s);
  else
    launch_nt<U, false>(a, grid, threads, nt_load, nt_store, s);
}

// ---- K3's access pattern on a chosen state layout (msp_adam_layout)
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

__device__ inline int64_t layout_tile(int64_t b, int64_t nb, int64_t chunk) {
  if (chunk <= 0) return b;
  const int64_t g0 = b / (8 * chunk) * (8 * chunk);
  const int64_t r = (nb - g0 < 8 * chunk) ? nb - g0 : 8 * chunk;
  const int64_t x = b % 8, xi = (b - g0) / 8, q = r / 8, rm = r % 8;
  return g0 + x * q + (x < rm ? x : rm) + xi;
}

__device__ inline float h2f(uint32_t w, int hi) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hi ? w >> 16 : w)));
}

__device__ inline uint32_t f2h2(float a, float b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(b))) << 16);
}

template <int T>
__global__ __launch_bounds__(128) void k_adam_layout(float* p0, float* m0, float* v0,
                                                     const uint32_t* g, uint32_t* copy,
                                                     int64_t n, int chunk) {
  const int64_t tile = layout_tile(blockIdx.x, gridDim.x, chunk);
  const int64_t i = tile * 512 + 4 * static_cast<int64_t>(threadIdx.x);
  if (i >= n) return;
  float *pp, *mp, *vp;
  if (T == 0) {
    pp = p0 + i;
    mp = m0 + i;
    vp = v0 + i;
  } else {
    pp = p0 + (i / T) * 3 * T + i % T;
    mp = pp + T;
    vp = pp + 2 * T;
  }
  const u2 gw = __builtin_nontemporal_load(reinterpret_cast<const u2*>(g + i / 2));
  f4 p = __builtin_nontemporal_load(reinterpret_cast<const f4*>(pp));
  f4 m = __builtin_nontemporal_load(reinterpret_cast<const f4*>(mp));
  f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4*>(vp));
  const float gv[4] = {h2f(gw[0], 0), h2f(gw[0], 1), h2f(gw[1], 0), h2f(gw[1], 1)};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    m[k] = __builtin_fmaf(gv[k], 0.1f, m[k] * 0.9f);
    v[k] = __builtin_fmaf(0.001f * gv[k], gv[k], v[k] * 0.999f);
    p[k] = p[k] + (-1e-3f * m[k]) / (sqrtf(v[k]) + 1e-8f);
  }
  __builtin_nontemporal_store(p, reinterpret_cast<f4*>(pp));
  __builtin_nontemporal_store(m, reinterpret_cast<f4*>(mp));
  __builtin_nontemporal_store(v, reinterpret_cast<f4*>(vp));
  __builtin_nontemporal_store(u2{f2h2(p[0], p[1]), f2h2(p[2], p[3])},
                              reinterpret_cast<u2*>(copy + i / 2));
}

}  // namespace

extern "C" {

int msp_abi_version(void) { return MSP_ABI_VERSION; }

int msp_stream(const void* const* rd, int32_t nread, void* const* wr, int32_t nwrite,
               int64_t nvec, int32_t threads, int32_t unroll, int32_t wave, int32_t grid,
               int32_t nt_load, int32_t nt_store, uint32_t* sink, void* stream) {
  if (nread < 0 || nread > MSP_MAX_ARRAYS || nwrite < 0 || nwrite > MSP_MAX_ARRAYS) return -1;
  if (nread + nwrite == 0 || nvec <= 0) return -1;
  if (threads < 64 || threads > kMaxThreads || threads % 64 != 0) return -1;
  if (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8) return -1;
  if (nwrite == 0 && sink == nullptr) return -1;
  ProbeArgs a = {};
  for (int k = 0; k < nread; ++k) {
    if (rd[k] == nullptr || (reinterpret_cast<uintptr_t>(rd[k]) & 15u)) return -1;
    a.rd[k] = static_cast<const u4*>(rd[k]);
  }
  for (int k = 0; k < nwrite; ++k) {
    if (wr[k] == nullptr || (reinterpret_cast<uintptr_t>(wr[k]) & 15u)) return -1;
    a.wr[k] = static_cast<u4*>(wr[k]);
  }
  a.nread = nread;
  a.nwrite = nwrite;
  a.nvec = nvec;
  a.sink = sink;
  const int64_t per_tile = static_cast<int64_t>(threads) * unroll;
  int64_t ntiles = (nvec + per_tile - 1) / per_tile;
  int64_t g = grid > 0 ? grid : ntiles;
  if (g > ntiles) g = ntiles;
  if (g > 0x7fffffff) g = 0x7fffffff;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (unroll) {
    case 1: launch_u<1>(a, static_cast<int>(g), threads, wave, nt_load, nt_store, s); break;
    case 2: launch_u<2>(a, static_cast<int>(g), threads, wave, nt_load, nt_store, s); break;
    case 4: launch_u<4>(a, static_cast<int>(g), threads, wave, nt_load, nt_store, s); break;
    default: launch_u<8>(a, static_cast<int>(g), threads, wave, nt_load, nt_store, s); break;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}

int msp_adam_layout(float* const* state, const void* g, void* copy, int64_t n,
                    int32_t interleave, int32_t xcd_chunk, void* stream) {
  if (state == nullptr || g == nullptr || copy == nullptr || n <= 0 || n % 512 != 0) return -1;
  if (interleave != 0 && interleave != 512 && interleave != 1024 && interleave != 2048 &&
      interleave != 4096)
    return -1;
  if (interleave != 0 && n % interleave != 0) return -1;
  if (xcd_chunk < 0 || n / 512 > 0x7fffffff) return -1;
  const int narr = interleave ? 1 : 3;
  for (int k = 0; k < narr; ++k)
    if (state[k] == nullptr || (reinterpret_cast<uintptr_t>(state[k]) & 15u)) return -1;
  if ((reinterpret_cast<uintptr_t>(g) & 7u) || (reinterpret_cast<uintptr_t>(copy) & 7u)) return -1;
  float* p = state[0];
  float* m = interleave ? state[0] : state[1];
  float* v = interleave ? state[0] : state[2];
  const auto* gw = static_cast<const uint32_t*>(g);
  auto* cw = static_cast<uint32_t*>(copy);
  const dim3 grid(static_cast<unsigned>(n / 512)), block(128);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (interleave) {
    case 0: hipLaunchKernelGGL(k_adam_layout<0>, grid, block, 0, s, p, m, v, gw, cw, n, xcd_chunk); break;
    case 512: hipLaunchKernelGGL(k_adam_layout<512>, grid, block, 0, s, p, m, v, gw, cw, n, xcd_chunk); break;
    case 1024: hipLaunchKernelGGL(k_adam_layout<1024>, grid, block, 0, s, p, m, v, gw, cw, n, xcd_chunk); break;
    case 2048: hipLaunchKernelGGL(k_adam_layout<2048>, grid, block, 0, s, p, m, v, gw, cw, n, xcd_chunk); break;
    default: hipLaunchKernelGGL(k_adam_layout<4096>, grid, block, 0, s, p, m, v, gw, cw, n, xcd_chunk); break;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}

}  // extern "C"
