// boundary.hip — gfx950 kernels of minispeed's gradient-accumulation
// boundary step and the C ABI declared in include/minispeed_boundary.h.
//
//   K1 k_grad_stats   ragged grad scan: inf/nan flag on the raw values,
//                     unscale (or a clip multiply), optional fp32 flat
//                     write, per-block fp64 sum of squares
//                                               (flat.py:196-257)
//   K2 k_norm_clip    deterministic second-level reduction, clip
//                     coefficient, skip flag, loss-scale update
//                                               (stage_1_and_2.py:105-128,
//                                                precision.py:50-92)
//   K3 k_adamw        fused clip + AdamW + master->model cast over the
//                     owned range              (optim/adam.py:59-93,
//                                                flat.py:133-154)
//   K4 k_cast         fp32 master -> model dtype (ZeRO-3 gather/free)
//   K5 k_accumulate   opt-in fp32 accumulation of one micro-batch gradient
//                     into its flat slice (contiguous gradients)
//
// Everything here is HBM-bound streaming; no MFMA.  Work is cut into tiles
// of consecutive flat indices.  In K3, K4 and K5 a lane moves quads of 4
// elements in wave order (see kStreamThreads), in K1 16-byte units of raw
// gradient in wave order.  A tile (K3-K5) or a segment piece (K1) with
// suitably aligned storage takes the vector path; tiles that straddle
// segment edges, partial tail tiles and misaligned segments take a
// per-element path.
//
// Arithmetic is written so that each rounding point of minispeed's torch op
// sequence is one IEEE fp32 operation here: the file is compiled with
// -ffp-contract=off, products/sums that torch fuses are explicit fmaf, and
// division and sqrt are the correctly rounded IEEE operations (HIP's
// default `/` and sqrtf lowering, not the native approximations).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>
#include <stdlib.h>

#include <mutex>

#include "minispeed_boundary.h"

// Slots of ms_boundary_scalars_noalloc: for each of MS_SCRATCH_MAX_GROUPS
// groups kStatsBlocksFixed fp64 partial sums, then as many uint32 flags, then
// MS_SCRATCH_MAX_TILES fp64 tile sums and as many uint32 tile flags (shared
// by the groups, which are scanned one after another).  Host code never
// names this array directly (its host-side name is not a device address):
// it uses the per-device address from hipGetSymbolAddress (scratch_base
// below).
#ifndef MS_STATS_BLOCKS
#define MS_STATS_BLOCKS 16384
#endif
constexpr int kStatsBlocksFixed = MS_STATS_BLOCKS;
static __device__ __align__(256) unsigned char scratch[
    (static_cast<size_t>(MS_SCRATCH_MAX_GROUPS) * kStatsBlocksFixed + MS_SCRATCH_MAX_TILES) *
    (sizeof(double) + sizeof(uint32_t))];

namespace {

// K3, K4 and K5 stream in "wave" order: a tile is T x U quads of 4
// consecutive elements (T threads, U quads per lane; kStreamThreads x
// kStreamUnroll for K4 and K5, kAdamThreads x kAdamUnroll for K3), and quad u
// of lane j is quad u * T + j, so every load or store instruction of a wave
// covers one contiguous run (64 x 16 bytes of fp32) and every cache line it
// touches is whole.  That is what lets every stream carry the non-temporal
// hint: with 8 consecutive elements per lane a store instruction writes
// half lines, and non-temporal half-line writes cost the fused AdamW ~40%.
#ifndef MS_STREAM_THREADS
#define MS_STREAM_THREADS 256
#endif
#ifndef MS_STREAM_UNROLL
#define MS_STREAM_UNROLL 2
#endif
constexpr int kStreamThreads = MS_STREAM_THREADS;
constexpr int kStreamUnroll = MS_STREAM_UNROLL;
constexpr int kStreamTile = kStreamThreads * kStreamUnroll * 4;   // 2048 flat elements (K4, K5)
// K3's own shape: one quad per lane, 512-element tiles.  Over the 1.3B
// state its K3 takes 5.77 ms against 5.79 ms with K4's 256 x 2 (the
// shard and the contiguous mode gain 1.5%), while K4 and K5 are 25-33%
// slower with K3's shape.
#ifndef MS_ADAM_THREADS
#define MS_ADAM_THREADS 128
#endif
#ifndef MS_ADAM_UNROLL
#define MS_ADAM_UNROLL 1
#endif
constexpr int kAdamThreads = MS_ADAM_THREADS;
constexpr int kAdamUnroll = MS_ADAM_UNROLL;
constexpr int kAdamTile = kAdamThreads * kAdamUnroll * 4;          // 512 flat elements (K3)
constexpr int kStatsBlocks = kStatsBlocksFixed;   // K2 partial slots per group
// K1, reading only: one wave scans a run of consecutive tiles of kScanTile
// flat indices (searching the segment table once and walking on with a
// cursor), several waves per block, a few 16-byte units of gradient in
// flight per lane.  Writing the fp32 flat gradient too: four waves per tile,
// one unit (two for fp32 gradients) per lane, the fp64 sum added up by one
// wave in the one-wave order.  Which waves scan a tile, and how many units
// they have in flight, do not change what K1 computes, so the shape is free
// per mode.  Over the 1.3B fp16 gradients (292 segments), in isolation:
// reading only, 8 waves x runs of 4 tiles x 4 units 0.398 ms (runs of
// 1 / 2 / 8: 0.59 / 0.43 / 0.43; 4 waves: 0.43; 2 units: 0.41; fp32
// gradients 0.822 ms, 2 units 0.841); writing, four waves per tile 1.25-1.27
// ms (one wave per tile x 2 units: 1.38; two slab sets and one barrier per
// tile: 1.26-1.28).
constexpr int kScanTile = MS_SCAN_TILE;
#ifndef MS_SCAN_WAVES_READ
#define MS_SCAN_WAVES_READ 8
#endif
#ifndef MS_SCAN_RUN_READ
#define MS_SCAN_RUN_READ 4
#endif
#ifndef MS_SCAN_DEPTH_READ
#define MS_SCAN_DEPTH_READ 4
#endif
// writing the flat gradient: one block per tile, its whole tiles split
// over the waves (fixed: 256 threads x 8 staged values = one tile); the
// other tiles, one wave walking them, one unit in flight per lane
#define MS_SCAN_WAVES_FLAT 4
#ifndef MS_SCAN_DEPTH_FLAT
#define MS_SCAN_DEPTH_FLAT 1
#endif
constexpr int kScanWavesRead = MS_SCAN_WAVES_READ;
constexpr int kScanWavesFlat = MS_SCAN_WAVES_FLAT;
// waves per SIMD K1 is compiled for: left alone, the compiler widens every
// unit of a round before the (serial) fp64 sum and needs 100+ VGPRs (4
// waves per SIMD); reading, held to 6 it keeps 56-72 (0.39-0.40 ms; with
// the walk before its ends were loaded early, 0.398 ms against 0.433 with
// 5 and 0.428 with 8); writing, 8 (1.27 ms against 1.40 with 6, where the
// walk of the other tiles took 80 VGPRs at 2 units per lane)
#ifndef MS_SCAN_MIN_WAVES
#define MS_SCAN_MIN_WAVES 6
#endif
#ifndef MS_SCAN_MIN_WAVES_FLAT
#define MS_SCAN_MIN_WAVES_FLAT 8
#endif
// Tiles per XCD in a row (xcd_tile) for K1 writing and K3: a K3-shaped
// stream over 1.3B elements takes 6.19-6.20 ms at 256-40000 against 6.40
// with block b on tile b (5.79 against 5.85 on a faster box); K3 itself,
// alternating runs on one box: 5.75-5.81 ms at 1024, 5.77-5.79 at 16384,
// 5.88-5.89 at 64
#ifndef MS_XCD_CHUNK
#define MS_XCD_CHUNK 1024
#endif
constexpr int64_t kXcdChunk = MS_XCD_CHUNK;
// Gradient bytes K1 leaves in the Infinity Cache (MALL, 256 MB on MI355X)
// for K3, which reads every gradient a second time.  K1's non-temporal loads
// do not keep what they read there; K3's non-temporal accesses of the
// masters, moments and model copy do not push out what is there.  So the
// reading K1 takes the runs of its last kCacheKeepBytes of gradient with
// ordinary loads (it reads them last, K3 reads them last) and K3 finds them
// in the cache.  Over the fp16 GPT lists, in bench steps on one box: 124M
// params 0.636 -> 0.618 ms, 350M 1.714 -> 1.694, 1.3B 6.228 -> 6.198 (K3
// 5.792 -> 5.763, K1 +6 us); 96 / 160 / 224 / 320 MiB / every run: 124M
// 0.634 / 0.627 / 0.619 / 0.620 / 0.619 ms, 1.3B 6.22 / 6.21 / 6.198 /
// 6.200 / 6.237 (ordinary loads throughout slow K1 by 40 us there).
#ifndef MS_CACHE_KEEP_MIB
#define MS_CACHE_KEEP_MIB 224
#endif
constexpr int64_t kCacheKeepBytes = int64_t(MS_CACHE_KEEP_MIB) << 20;
constexpr int kNormThreads = 1024;        // K2 block: 16 wave64
static_assert(kStatsBlocks % kNormThreads == 0, "K2 takes the same number of partials per thread");
constexpr int kMaxSegs = 1 << 26;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// Address-space qualifiers for pointers the compiler cannot classify on its
// own (addresses read from segment tables or kept in structs): global
// memory and LDS accesses then compile to global_* / ds_* instructions
// instead of generic flat_* ones, which also count against the
// scalar-load counter and so lengthen every wait on a scalar load.
#define MS_GLOBAL __attribute__((address_space(1)))
#define MS_LDS __attribute__((address_space(3)))

// ---------------------------------------------------------------- dtypes
// Raw storage <-> fp32.  Widening is exact; narrowing rounds to nearest
// even (torch's fp32 -> fp16/bf16 copy_).  The inf/nan test looks at the
// exponent field of the stored value, so every NaN payload and both
// infinities count, exactly like torch.isfinite on the widened value.
struct DF32 {
  using raw = uint32_t;
  static constexpr int kBytes = 4;
  // packed inf/nan test: ((w & kExp) + kExpOne) sets bit 31 exactly when
  // the exponent field is all ones
  static constexpr uint32_t kExp = 0x7f800000u, kExpOne = 0x00800000u,
                            kTop = 0x80000000u;
  __device__ static float widen(raw r) { return __uint_as_float(r); }
  __device__ static bool nonfinite(raw r) {
    return (r & 0x7f800000u) == 0x7f800000u;
  }
  __device__ static raw narrow(float f) { return __float_as_uint(f); }
};

struct DF16 {
  using raw = uint16_t;
  static constexpr int kBytes = 2;
  // per 16-bit half: the add carries into the half's top bit exactly when
  // its exponent field is all ones, and never into the next half
  static constexpr uint32_t kExp = 0x7c007c00u, kExpOne = 0x04000400u,
                            kTop = 0x80008000u;
  __device__ static float widen(raw r) {
    return static_cast<float>(__builtin_bit_cast(_Float16, r));
  }
  __device__ static bool nonfinite(raw r) { return (r & 0x7c00u) == 0x7c00u; }
  __device__ static raw narrow(float f) {
    return __builtin_bit_cast(raw, static_cast<_Float16>(f));
  }
};

struct DBF16 {
  using raw = uint16_t;
  static constexpr int kBytes = 2;
  static constexpr uint32_t kExp = 0x7f807f80u, kExpOne = 0x00800080u,
                            kTop = 0x80008000u;
  __device__ static float widen(raw r) {
    return __uint_as_float(static_cast<uint32_t>(r) << 16);
  }
  __device__ static bool nonfinite(raw r) { return (r & 0x7f80u) == 0x7f80u; }
  __device__ static raw narrow(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<raw>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<raw>(u >> 16);
  }
};

// 16 bytes of raw gradient (8 fp16 / bf16 or 4 fp32 elements), 16-byte
// aligned, as four 32-bit words: with the non-temporal hint, or (kKeep) as
// an ordinary load, which leaves the lines in the Infinity Cache for K3
// (kCacheKeepBytes below).
template <bool kKeep = false>
__device__ inline void load_unit(const void* p, uint32_t (&w)[4]) {
  u4 x;
  if constexpr (kKeep)
    x = *((const MS_GLOBAL u4*)p);
  else
    x = __builtin_nontemporal_load((const MS_GLOBAL u4*)p);
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = x[k];
}

template <class D>
__device__ inline typename D::raw unit_elem(const uint32_t (&w)[4], int k) {
  if constexpr (D::kBytes == 2)
    return static_cast<uint16_t>((k & 1) ? (w[k >> 1] >> 16) : (w[k >> 1] & 0xffffu));
  else
    return w[k];
}

// A quad: 4 consecutive elements, 16 bytes of fp32 or 8 of fp16 / bf16, at an
// address aligned to its size.  Every K3 / K4 stream is touched once per
// element (read, then written back once) and moves through these with the
// non-temporal hint.
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

__device__ inline void ldq(const float* p, float (&x)[4]) {
  const f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
  x[0] = v[0];
  x[1] = v[1];
  x[2] = v[2];
  x[3] = v[3];
}

__device__ inline void stq(float* p, const float (&x)[4]) {
  __builtin_nontemporal_store(f4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f4*>(p));
}

template <class D>
__device__ inline void widen_words(uint32_t w0, uint32_t w1, float (&x)[4]) {
  x[0] = D::widen(static_cast<uint16_t>(w0 & 0xffffu));
  x[1] = D::widen(static_cast<uint16_t>(w0 >> 16));
  x[2] = D::widen(static_cast<uint16_t>(w1 & 0xffffu));
  x[3] = D::widen(static_cast<uint16_t>(w1 >> 16));
}

template <class D>
__device__ inline void narrow_words(const float (&x)[4], uint32_t& w0, uint32_t& w1) {
  w0 = static_cast<uint32_t>(D::narrow(x[0])) | (static_cast<uint32_t>(D::narrow(x[1])) << 16);
  w1 = static_cast<uint32_t>(D::narrow(x[2])) | (static_cast<uint32_t>(D::narrow(x[3])) << 16);
}

// A quad of raw storage (fp16 / bf16 / fp32) at a quad-aligned address
// (generic pointers, flat_* instructions: K3 over 1.3B params 5.75-5.81 ms
// against 5.81-5.82 with global_* ones, alternating runs on one box).
template <class D>
__device__ inline void ldq_raw(const void* p, float (&x)[4]) {
  if constexpr (D::kBytes == 2) {
    const u2 w = __builtin_nontemporal_load(reinterpret_cast<const u2*>(p));
    widen_words<D>(w[0], w[1], x);
  } else {
    ldq(static_cast<const float*>(p), x);
  }
}

template <class D>
__device__ inline void stq_raw(void* p, const float (&x)[4]) {
  if constexpr (D::kBytes == 2) {
    uint32_t w0, w1;
    narrow_words<D>(x, w0, w1);
    __builtin_nontemporal_store(u2{w0, w1}, reinterpret_cast<u2*>(p));
  } else {
    stq(static_cast<float*>(p), x);
  }
}

// `p` advanced by `elems` elements of `bytes` each is aligned for a quad
__device__ inline bool quad_aligned(const void* p, int64_t elems, int bytes) {
  return ((reinterpret_cast<uintptr_t>(p) + static_cast<uintptr_t>(elems * bytes)) &
          static_cast<uintptr_t>(4 * bytes - 1)) == 0;
}

// Quads anywhere an element can be.  Flat layouts pack tensors back to back,
// so one tensor of odd size puts every later gradient and model copy off
// the quad alignment of the flat tiles.  kind 0: aligned to the quad;
// kind 1: 4-byte aligned (one access of 4-byte alignment, which global
// memory takes for multi-dword loads and stores); kind 2: 2 mod 4 (2-byte
// elements only), loaded as the three words around the quad (ldq_any) and
// stored a whole run of quads at a time as 8-byte aligned words passed
// between neighbouring lanes (stq_run_kind2, below).
typedef float f4w __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u2w __attribute__((ext_vector_type(2), aligned(4)));

template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

__device__ inline int quad_kind(const void* p, int64_t elems, int bytes) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p) + static_cast<uintptr_t>(elems * bytes);
  if ((a & static_cast<uintptr_t>(4 * bytes - 1)) == 0) return 0;
  return (a & 3u) == 0 ? 1 : 2;
}

template <class D>
__device__ inline void ldq_any(const void* p, int kind, float (&x)[4]) {
  if (kind == 0) {
    ldq_raw<D>(p, x);
  } else if constexpr (D::kBytes == 4) {
    const f4w v = __builtin_nontemporal_load((const MS_GLOBAL f4w*)p);
    x[0] = v[0];
    x[1] = v[1];
    x[2] = v[2];
    x[3] = v[3];
  } else if (kind == 1) {
    const u2w w = __builtin_nontemporal_load((const MS_GLOBAL u2w*)p);
    widen_words<D>(w[0], w[1], x);
  } else {
    // kind 2: the three words around the quad, one element before and one
    // after it included (inside the tensor where the caller checked it),
    // joined with alignbit.  (Whole words passed between neighbouring lanes,
    // as the stores do, took K3 over the shifted 1.3B list from 5.88-5.91
    // to 6.03-6.05 ms: each lane's shuffle waits for its load.)
    const MS_GLOBAL uint32_t* q = (const MS_GLOBAL uint32_t*)(static_cast<const char*>(p) - 2);
    const u2w lo = __builtin_nontemporal_load((const MS_GLOBAL u2w*)q);
    const uint32_t hi = __builtin_nontemporal_load(q + 2);
    widen_words<D>(__builtin_amdgcn_alignbit(lo[1], lo[0], 16),
                   __builtin_amdgcn_alignbit(hi, lo[1], 16), x);
  }
}

// kinds 0 and 1 (kind 2 of a 2-byte type: stq_run_kind2)
template <class D>
__device__ inline void stq_any(void* p, int kind, const float (&x)[4]) {
  if (kind == 0) {
    stq_raw<D>(p, x);
  } else if constexpr (D::kBytes == 4) {
    __builtin_nontemporal_store(f4w{x[0], x[1], x[2], x[3]}, (MS_GLOBAL f4w*)p);
  } else {   // kind 1
    uint32_t w0, w1;
    narrow_words<D>(x, w0, w1);
    __builtin_nontemporal_store(u2w{w0, w1}, (MS_GLOBAL u2w*)p);
  }
}

// The kind-2 stores of a run of kThreads consecutive quads of a 2-byte type,
// quad j of the run held by thread j (K3's and K4's wave order), the run's
// first element 2 mod 4 bytes off.  Stored quad by quad (2 + 4 + 2 bytes per
// lane) every store instruction of a wave writes parts of lines: K3 over the
// shifted 1.3B GPT list took 6.01 ms against 5.88-5.91 this way (aligned
// list: 5.75).  Instead lane j joins the last 4 - s elements of its quad
// with the first s of lane j + 1's into the 8-byte aligned word that starts
// at the run's element 4j + s (s = 1 or 3: the elements before the first
// 8-byte boundary), so a wave's store covers a contiguous run of whole
// lines.  Within a wave the neighbour's quad comes by a shuffle; across a
// wave boundary through `xq` (LDS, two words per wave of the block): the
// first lane of each later wave hands its quad to the previous wave's last
// lane, so the line at a wave boundary is written whole by one wave, not in
// two pieces (the memory completes a partial line by reading it first: K3
// on the shifted list 5.85-5.88 ms with the pieces, 5.70-5.72 ms without).
// Only the run's ends go as single elements: the last 4 - s of the run's
// last lane and the first s of its first lane.  Every element of the run is
// written once; nothing outside it is touched.  All threads of the block
// call this together (it holds a barrier); consecutive calls alternate
// between two `xq` buffers, so a wave that runs ahead does not overwrite a
// hand-over before it is read.
template <class D, int kThreads>
__device__ inline void stq_run_kind2(void* run, int j, const float (&x)[4],
                                     MS_LDS uint32_t* __restrict__ xq) {
  static_assert(D::kBytes == 2, "2-byte types only");
  uint32_t w0, w1;
  narrow_words<D>(x, w0, w1);
  const int s = static_cast<int>(((8u - (reinterpret_cast<uintptr_t>(run) & 7u)) & 7u) >> 1);
  uint32_t n0 = __shfl_down(w0, 1u, 64), n1 = __shfl_down(w1, 1u, 64);
  const int wl = j & 63;
  if (wl == 0 && j != 0) {
    xq[2 * ((j >> 6) - 1)] = w0;
    xq[2 * ((j >> 6) - 1) + 1] = w1;
  }
  __syncthreads();
  if (wl == 63 && j != kThreads - 1) {
    n0 = xq[2 * (j >> 6)];
    n1 = xq[2 * (j >> 6) + 1];
  }
  const uint64_t q = (static_cast<uint64_t>(w1) << 32) | w0;
  const uint64_t qn = (static_cast<uint64_t>(n1) << 32) | n0;
  MS_GLOBAL uint16_t* e = (MS_GLOBAL uint16_t*)run + 4 * j;   // the quad's first element
  if (j != kThreads - 1) {
    const uint64_t word = (q >> (16 * s)) | (qn << (16 * (4 - s)));
    __builtin_nontemporal_store(word, (MS_GLOBAL uint64_t*)(e + s));
  } else {
    for (int k = s; k < 4; ++k)
      __builtin_nontemporal_store(static_cast<uint16_t>(q >> (16 * k)), e + k);
  }
  if (j == 0) {
    for (int k = 0; k < s; ++k)
      __builtin_nontemporal_store(static_cast<uint16_t>(q >> (16 * k)), e + k);
  }
}

// LDS of stq_run_kind2's hand-overs for a block of kThreads: two buffers of
// two words per wave
template <int kThreads>
struct Kind2Lds {
  uint32_t w[2][2 * (kThreads / 64)];
};

template <class D>
__device__ inline typename D::raw load_raw1(const void* base, int64_t k) {
  return ((const MS_GLOBAL typename D::raw*)base)[k];
}

template <class D>
__device__ inline void store_raw1(void* base, int64_t k, typename D::raw v) {
  ((MS_GLOBAL typename D::raw*)base)[k] = v;
}

__device__ inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Largest s with segs[s].begin <= i (segs sorted, segs[0].begin <= i).
__device__ inline int find_seg(const ms_segment_t* segs, int nseg, int64_t i) {
  int lo = 0, hi = nseg - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (segs[mid].begin <= i)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

__device__ inline int64_t seg_end(const ms_segment_t& s) {
  return s.begin + s.numel;
}

// The tile block b of nb starts on.  Blocks are dealt to the 8 XCDs in
// turn (block b to XCD b % 8), each XCD with its own L2.  Blocks go in
// groups of 8 * chunk (the last one may be shorter, r blocks); the r tiles
// of a group are split into 8 contiguous runs, run x (r / 8 tiles, one more
// for x < r % 8) for the blocks of XCD x in order.  A bijection of [0, nb)
// for any nb >= 1 and chunk >= 1.
__device__ inline int64_t xcd_tile(int64_t b, int64_t nb, int64_t chunk) {
  const int64_t g0 = b / (8 * chunk) * (8 * chunk);
  const int64_t r = (nb - g0 < 8 * chunk) ? nb - g0 : 8 * chunk;
  const int64_t x = b % 8, xi = (b - g0) / 8, q = r / 8, rm = r % 8;
  return g0 + x * q + (x < rm ? x : rm) + xi;
}

// Loss-scale division.  mode 0: none; 1: multiply by the exact reciprocal of
// a power-of-two scale (x / 2^k and x * 2^-k round identically, subnormal
// results included); 2: IEEE division; 3: one rounded multiply by `scale`
// (the clip coefficient of scale_grads, flat.py:249-257).
__device__ inline float unscale1(float g, int mode, float scale, float inv) {
  if (mode == 1) return g * inv;
  if (mode == 2) return g / scale;
  if (mode == 3) return g * scale;
  return g;
}

// ------------------------------------------------------- block reductions
__device__ inline double wave_sum(double x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// ------------------------------------------------------------------ K1
// One wave scans one tile [r0, r1) of kScanTile flat indices, walking the
// segments inside it with a cursor.  Each piece of a segment is a scalar
// head, a vector body of 16-byte units (lane l takes units l, l + 64, ...)
// and a scalar tail; which path a piece takes depends only on the segment
// (its gradient's alignment), never on whether the flat gradient is
// written, so both modes give the same statistics bit for bit.  Lanes
// accumulate their own elements in index order and the wave reduces with a
// fixed xor tree, so a tile's partial is a pure function of the layout.
//
// Tiles of consecutive waves are adjacent, so the waves resident at any
// moment read and write one compact window of the flat range; a block per
// contiguous 1/16384 of the range instead (each resident block streaming
// its own distant range) wrote the fp32 flat gradient at 4.5 TB/s against
// 5.8 TB/s this way.

// K1's scaling of the widened gradient, fixed per launch: none, one rounded
// multiply by `mul` (the exact reciprocal of a power-of-two loss scale, or
// scale_grads' factor; unscale1 modes 1 and 3) or IEEE division by `div`
// (mode 2).  A compile-time choice keeps the per-element path free of
// branches, so the widened units of a round need not all be held at once.
enum { kScaleNone = 0, kScaleMul = 1, kScaleDiv = 2 };

template <int kScale>
__device__ inline float scale_grad(float g, float mul, float div) {
  if constexpr (kScale == kScaleMul) return g * mul;
  else if constexpr (kScale == kScaleDiv) return g / div;
  else return g;
}

// kSumFlags: the inf/nan flag of the counted elements' 16-byte units comes
// from their fp64 sum of squares instead of a test of every word.  Exact
// when the scaling cannot turn a finite gradient into inf (none, a multiply
// by a factor in [-1, 1], a division by at least 1): an inf/nan element then squares
// to inf/nan and the sum is inf/nan, while finite elements (fp32 at most
// 3.4e38) square and add up to at most ~1e81 in fp64; the sum of squares is
// non-negative, so inf never meets -inf.  Elements outside the owned range
// (not counted) are still tested one by one.
template <class G, bool kFlat, bool kStats, int kScale, bool kKeep = false,
          bool kSumFlags = false>
struct GradScan {
  static_assert(!kSumFlags || kStats, "the flags come from the statistics");
  static constexpr bool kFlagsFromSum = kSumFlags;
  static constexpr int kScanDepth = kFlat ? MS_SCAN_DEPTH_FLAT : MS_SCAN_DEPTH_READ;
  static constexpr int kUnit = 16 / G::kBytes;   // elements per 16-byte unit
  float mul, div;
  int64_t begin;
  MS_GLOBAL float* flat;
  double acc = 0.0;
  bool bad = false;      // per-element inf/nan tests
  uint32_t packed = 0;   // packed exponent tests of the vector body

  // element i, its raw value r already loaded (ignored where sg.grad is
  // null: a zero)
  template <bool kCount>
  __device__ void use1(const ms_segment_t& sg, int64_t i, typename G::raw r) {
    float g = 0.0f;
    if (sg.grad) {
      bad |= G::nonfinite(r);
      g = scale_grad<kScale>(G::widen(r), mul, div);
    }
    if (kStats && kCount) {
      const double d = static_cast<double>(g);
      acc = __builtin_fma(d, d, acc);
    }
    if (kFlat) flat[i - begin] = g;
  }

  template <bool kCount>
  __device__ void element(const ms_segment_t& sg, int64_t i) {
    use1<kCount>(sg, i, sg.grad ? load_raw1<G>(sg.grad, i - sg.begin) : typename G::raw(0));
  }

  // One unit: the 16 bytes of raw gradient a lane moves with one load, as
  // four 32-bit words, widened (and counted) into g.
  template <bool kCount>
  __device__ void widen(const uint32_t (&w)[4], float (&g)[kUnit]) {
    if constexpr (!(kSumFlags && kCount && kStats)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) packed |= (w[j] & G::kExp) + G::kExpOne;
    }
#pragma unroll
    for (int k = 0; k < kUnit; ++k) {
      g[k] = scale_grad<kScale>(G::widen(unit_elem<G>(w, k)), mul, div);
      if (kStats && kCount) {
        const double d = static_cast<double>(g[k]);
        acc = __builtin_fma(d, d, acc);
      }
    }
  }

  // g -> flat indices i .. i + kUnit - 1; fvec: that range is 16-byte aligned
  __device__ void put(const float (&g)[kUnit], int64_t i, bool fvec) {
    MS_GLOBAL float* o = flat + (i - begin);
    if (fvec) {
#pragma unroll
      for (int k = 0; k < kUnit; k += 4)
        __builtin_nontemporal_store(f4{g[k], g[k + 1], g[k + 2], g[k + 3]},
                                    (MS_GLOBAL f4*)(o + k));
    } else {
#pragma unroll
      for (int k = 0; k < kUnit; ++k) o[k] = g[k];
    }
  }

  // elements [a, b) of segment sg, all inside (kCount) or all outside the
  // owned range
  template <bool kCount>
  __device__ void piece(const ms_segment_t& sg, int64_t a, int64_t b, int lane) {
    const bool vec = sg.grad != nullptr && aligned16(sg.grad);
    if (!vec) {
      if (!sg.grad && !kFlat) return;      // zeros: nothing to count or test
      for (int64_t i = a + lane; i < b; i += 64) element<kCount>(sg, i);
      return;
    }
    const int64_t au = sg.begin + (((a - sg.begin) + kUnit - 1) & ~int64_t(kUnit - 1));
    const int64_t bu = sg.begin + ((b - sg.begin) & ~int64_t(kUnit - 1));
    if (au >= bu) {
      for (int64_t i = a + lane; i < b; i += 64) element<kCount>(sg, i);
      return;
    }
    // The head [a, au) and the tail [bu, b) hold fewer than kUnit elements
    // each: one per lane at most.  Each lane adds its head element, its
    // tail element, then its units.  Reading only, the two elements are
    // loaded first and added after the first body loads are issued, so a
    // piece costs one memory round trip, not three; writing (the tiles the
    // split paths of k_grad_stats leave to the walk: segment edges, missing
    // gradients, storage off 16 bytes) they are added first,
    // which keeps the registers of that kernel, compiled for 8 waves per
    // SIMD, within bounds.
    const int64_t hi = a + lane, ti = bu + lane;
    const bool hv = hi < au, tv = ti < b;
    typename G::raw hr = 0, tr = 0;
    if constexpr (kFlat) {
      if (hv) element<kCount>(sg, hi);
      if (tv) element<kCount>(sg, ti);
    } else {
      if (hv) hr = load_raw1<G>(sg.grad, hi - sg.begin);
      if (tv) tr = load_raw1<G>(sg.grad, ti - sg.begin);
    }
    bool ends = !kFlat;   // per lane: added before the lane's first unit
    auto add_ends = [&] {
      if (ends) {
        if (hv) use1<kCount>(sg, hi, hr);
        if (tv) use1<kCount>(sg, ti, tr);
        ends = false;
      }
    };
    const int64_t nu = (bu - au) / kUnit;
    const char* src = static_cast<const char*>(sg.grad) + (au - sg.begin) * G::kBytes;
    const bool fvec = kFlat && aligned16((const void*)(flat + (au - begin)));
    // Wave order: lane l takes units l, l + 64, ..., so each load
    // instruction of the wave reads one contiguous kilobyte of whole cache
    // lines.  A round has up to kScanDepth units in flight per lane (fewer
    // at the end of the piece: a lane's last round is partial, never a
    // string of single units); each lane still takes its units in
    // increasing order, so its running sum does not depend on the depth or
    // on the mode.
    for (int64_t u = lane; u < nu; u += kScanDepth * 64) {
      uint32_t w[kScanDepth][4];
#pragma unroll
      for (int d = 0; d < kScanDepth; ++d)
        if (u + d * 64 < nu) load_unit<kKeep>(src + (u + d * 64) * 16, w[d]);
      add_ends();
#pragma unroll
      for (int d = 0; d < kScanDepth; ++d) {
        if (u + d * 64 < nu) {
          float g[kUnit];
          widen<kCount>(w[d], g);
          if (kFlat) put(g, au + (u + d * 64) * kUnit, fvec);
        }
      }
    }
    add_ends();
  }
};

template <bool kFlat>
constexpr int scan_waves() { return kFlat ? kScanWavesFlat : kScanWavesRead; }
template <bool kFlat>
constexpr int scan_min_waves() { return kFlat ? MS_SCAN_MIN_WAVES_FLAT : MS_SCAN_MIN_WAVES; }

// Writing the flat gradient: a whole tile [r0, r0 + kScanTile) of one
// segment whose first element sits m (> 0) elements into a 16-byte unit of
// the (16-byte aligned) storage, so that the tile is a head of nh = kUnit -
// m elements, kScanTile / kUnit - 1 whole units and a tail of m elements —
// the pieces the walk of scan_tile takes.  All the block's waves load the
// units (lane l of wave w: units (w * kPerLane + k) * 64 + l) and stage the
// widened values in tile order at F[kUnit - nh + i], which puts every unit
// on a 16-byte boundary of F; wave 0 loads the head, wave 1 the tail.
// After the barrier every wave writes 512 consecutive floats of the tile,
// one float per lane and store (64 consecutive floats, whole lines), and
// wave 0 adds the squares in the walk's order: lane l its head element,
// its tail element, then units l, l + 64, ..., so the slot gets the bits
// one wave alone gives it.
template <class Scan, class G, bool kStats, int kScale, int kWaves>
__device__ void split_tile_shifted(Scan& sc, const ms_segment_t& sg, int64_t r0, int64_t begin,
                                   int m, bool owned, float* __restrict__ flat, int64_t t,
                                   double* __restrict__ tsum, uint32_t* __restrict__ tflag,
                                   MS_LDS float* F, MS_LDS uint32_t* wflag, int wave, int lane,
                                   float mul, float div) {
  constexpr int kUnit = Scan::kUnit;
  constexpr int kUnits = kScanTile / kUnit - 1;          // whole units of the tile
  constexpr int kPerLane = (kUnits + 64 * kWaves) / (64 * kWaves);
  static_assert(kPerLane * 64 * kWaves == kUnits + 1, "one unit slot per lane and round");
  static_assert(kWaves >= 2, "wave 0 loads the head, wave 1 the tail");
  const int nh = kUnit - m;
  const int off = kUnit - nh;                            // F index of tile element 0
  const int64_t e0 = r0 - sg.begin;                      // storage element of tile element 0
  const char* usrc = static_cast<const char*>(sg.grad) + (e0 + nh) * G::kBytes;
  uint32_t w[kPerLane][4];
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) {
    const int u = (wave * kPerLane + k) * 64 + lane;
    if (u < kUnits) load_unit(usrc + static_cast<int64_t>(u) * 16, w[k]);
  }
  // head (wave 0, lanes < nh) and tail (wave 1, lanes < m) elements
  bool ebad = false;
  const bool head = wave == 0 && lane < nh, tail = wave == 1 && lane < m;
  if (head || tail) {
    const int64_t e = head ? e0 + lane : e0 + kScanTile - m + lane;
    const typename G::raw r = load_raw1<G>(sg.grad, e);
    ebad = G::nonfinite(r);
    F[head ? off + lane : kScanTile + lane] = scale_grad<kScale>(G::widen(r), mul, div);
  }
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) {
    const int u = (wave * kPerLane + k) * 64 + lane;
    if (u < kUnits) {
      float g[kUnit];
      sc.template widen<false>(w[k], g);
      MS_LDS f4* d = (MS_LDS f4*)(F + kUnit * (u + 1));
#pragma unroll
      for (int q = 0; q < kUnit / 4; ++q) d[q] = f4{g[4 * q], g[4 * q + 1], g[4 * q + 2], g[4 * q + 3]};
    }
  }
  if constexpr (kStats) {
    const bool wb = __any(ebad || (sc.packed & G::kTop) != 0);
    if (lane == 0) wflag[wave] = wb ? 1u : 0u;
  }
  __syncthreads();
  MS_GLOBAL float* o = (MS_GLOBAL float*)flat + (r0 - begin);
  constexpr int kPerWave = kScanTile / kWaves;
#pragma unroll
  for (int i = 0; i < kPerWave / 64; ++i) {
    const int p = wave * kPerWave + i * 64 + lane;
    __builtin_nontemporal_store(F[off + p], o + p);
  }
  if constexpr (kStats) {
    if (wave == 0) {
      double acc = 0.0;
      if (owned) {
        auto add = [&](float v) {
          const double x = static_cast<double>(v);
          acc = __builtin_fma(x, x, acc);
        };
        if (lane < nh) add(F[off + lane]);
        if (lane < m) add(F[kScanTile + lane]);
#pragma unroll 1
        for (int u = lane; u < kUnits; u += 64) {
          const MS_LDS f4* d = (const MS_LDS f4*)(F + kUnit * (u + 1));
#pragma unroll
          for (int q = 0; q < kUnit / 4; ++q) {
            const f4 x = d[q];
            add(x[0]);
            add(x[1]);
            add(x[2]);
            add(x[3]);
          }
        }
      }
      const double tot = wave_sum(acc);
      if (lane == 0) {
        uint32_t f = 0;
#pragma unroll
        for (int d = 0; d < kWaves; ++d) f |= wflag[d];
        tsum[t] = tot;
        tflag[t] = f;
      }
    }
  }
}

// Tile t = [r0, r1) by one wave: walk its segments from the cursor s (left
// on the segment that holds r1 when that one goes on), then the tile's
// statistics into its slot.
template <class Scan, class G, bool kStats>
__device__ void scan_tile(Scan& sc, const ms_segment_t* segs, int nseg, int& s, int64_t t,
                          int64_t r0, int64_t r1, int64_t own_begin, int64_t own_end,
                          double* tsum, uint32_t* tflag, int lane) {
  for (; s < nseg; ++s) {
    const ms_segment_t sg = segs[s];
    const int64_t se = seg_end(sg);
    const int64_t a = sg.begin > r0 ? sg.begin : r0;
    const int64_t b = se < r1 ? se : r1;
    if (a < b) {
      // split at the owned range so every piece is counted or not
      const int64_t o0 = own_begin > a ? (own_begin < b ? own_begin : b) : a;
      const int64_t o1 = own_end < b ? (own_end > o0 ? own_end : o0) : b;
      if (a < o0) sc.template piece<false>(sg, a, o0, lane);
      if (o0 < o1) sc.template piece<kStats>(sg, o0, o1, lane);
      if (o1 < b) sc.template piece<false>(sg, o1, b, lane);
    }
    if (se > r1) break;   // it also holds the next tile's first index
  }
  if (kStats) {
    bool bad = sc.bad || (sc.packed & G::kTop) != 0;
    if constexpr (Scan::kFlagsFromSum) bad = bad || !__builtin_isfinite(sc.acc);
    const double w = wave_sum(sc.acc);
    const bool wb = __any(bad);
    if (lane == 0) {
      tsum[t] = w;
      tflag[t] = wb ? 1u : 0u;
    }
  }
}

// Reading only (kFlat false): each wave scans runs of `run` consecutive
// tiles; a run starting at tile keep_from or later is loaded with ordinary
// loads (kCacheKeepBytes).  Writing the flat gradient (kFlat): one block of kScanWavesFlat
// waves per tile.  A whole tile inside one segment with 16-byte aligned
// storage, starting on a unit boundary of it and owned or not as a whole,
// is split across the waves: wave w loads, widens and writes units
// w*k*64 + lane .. (k units per lane), each store covering whole lines; the
// widened values wait in LDS, and after a barrier wave 0 adds each lane's
// units l, l + 64, ... in index order — the order one wave scanning the
// tile alone uses, so the slots get the same bits.  Such a tile starting
// inside a unit of its storage is split the same way with its head and
// tail elements (split_tile_shifted).  Any other tile is scanned by wave 0
// alone, as when reading.
template <class G, bool kFlat, bool kStats, int kScale, bool kSumFlags = false>
__global__ __launch_bounds__(64 * scan_waves<kFlat>(), scan_min_waves<kFlat>()) void k_grad_stats(
    const ms_segment_t* __restrict__ segs, int nseg, int64_t begin,
    int64_t end, int64_t own_begin, int64_t own_end, float mul, float div,
    float* __restrict__ flat, double* __restrict__ tsum, uint32_t* __restrict__ tflag,
    int64_t ntiles, int run, int64_t keep_from) {
  static_assert(!(kFlat && kSumFlags), "writing, the flags come from the per-word tests");
  constexpr int kWaves = scan_waves<kFlat>();
  using Scan = GradScan<G, kFlat, kStats, kScale>;
  // writing: a tile's widened values (aligned tiles: one slab of 128 f4
  // per wave; tiles off the storage's unit grid: the tile in order from
  // float kUnit - head, which takes up to 8 floats of the last row)
  __shared__ f4 slabs[kFlat ? kWaves + 1 : 1][128];
  const int lane = threadIdx.x & 63;
  // uniform across the wave, and known to be so by the compiler: the tile
  // bounds, the segment search and the piece bookkeeping stay scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if constexpr (!kFlat) {
    // a wave's tiles are uniform across it: no block-level barrier
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kWaves * run;
    for (int64_t t0 = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * run; t0 < ntiles;
         t0 += stride) {
      const int64_t t1 = (t0 + run < ntiles) ? t0 + run : ntiles;
      // the cursor: the segment holding the next tile's first index
      int s = find_seg(segs, nseg, begin + t0 * kScanTile);
      // the run's load hint, a compile-time choice (a runtime one merges
      // the two loads into one without the hint)
      auto scan_run = [&](auto keep) {
        using S = GradScan<G, kFlat, kStats, kScale, decltype(keep)::value, kSumFlags>;
        for (int64_t t = t0; t < t1; ++t) {
          S sc;
          sc.mul = mul;
          sc.div = div;
          sc.begin = begin;
          sc.flat = (MS_GLOBAL float*)flat;
          const int64_t r0 = begin + t * kScanTile;
          const int64_t r1 = (r0 + kScanTile < end) ? r0 + kScanTile : end;
          scan_tile<S, G, kStats>(sc, segs, nseg, s, t, r0, r1, own_begin, own_end, tsum,
                                  tflag, lane);
        }
      };
      if (t0 >= keep_from)
        scan_run(BoolC<true>{});
      else
        scan_run(BoolC<false>{});
    }
  } else {
    constexpr int kUnit = Scan::kUnit;
    constexpr int kPerLane = kScanTile / kUnit / (64 * kWaves);   // 1 (2-byte) or 2 (4-byte)
    static_assert(kPerLane * kUnit == 8, "each lane stages 8 widened values of a tile");
    __shared__ uint32_t wflag[kWaves];
    // tiles are uniform across the block, and so are its barriers
    // XCD-ordered: neighbouring tiles' 12-byte slots leave the same L2 as
    // whole lines (tile t in block t would write every slot as two partial
    // lines from two L2s: +40 MB of writes at 1.3B)
    const int64_t tfirst = xcd_tile(blockIdx.x, gridDim.x, kXcdChunk);
    // the segment holding the block's next tile: searched for while the
    // current tile's loads are in flight (a block takes its tiles one after
    // another, so the search would otherwise add to every tile's time)
    int snext = tfirst < ntiles ? find_seg(segs, nseg, begin + tfirst * kScanTile) : 0;
    for (int64_t t = tfirst; t < ntiles; t += gridDim.x) {
      Scan sc;
      sc.mul = mul;
      sc.div = div;
      sc.begin = begin;
      sc.flat = (MS_GLOBAL float*)flat;
      const int64_t r0 = begin + t * kScanTile;
      const int64_t r1 = (r0 + kScanTile < end) ? r0 + kScanTile : end;
      int s = snext;
      const ms_segment_t sg = segs[s];
      const bool owned = own_begin <= r0 && r1 <= own_end;
      // a whole tile inside one segment, storage and flat output 16-byte
      // aligned, owned or not as a whole
      const bool split = r1 - r0 == kScanTile && sg.grad != nullptr && aligned16(sg.grad) &&
                         sg.begin <= r0 && r1 <= seg_end(sg) &&
                         aligned16((const void*)(flat + (r0 - begin))) &&
                         (owned || r1 <= own_begin || own_end <= r0);
      const int64_t tn = t + gridDim.x;
      if (!split) {
        // the other tiles (segment edges, missing gradients, storage off
        // 16 bytes): wave 0 walks them as when reading
        if (wave == 0)
          scan_tile<Scan, G, kStats>(sc, segs, nseg, s, t, r0, r1, own_begin, own_end, tsum,
                                     tflag, lane);
        if (tn < ntiles) snext = find_seg(segs, nseg, begin + tn * kScanTile);
        continue;
      }
      // the tile's first element sits m elements into a unit of the storage
      const int m = static_cast<int>((r0 - sg.begin) & (kUnit - 1));
      if (m != 0) {
        split_tile_shifted<Scan, G, kStats, kScale, kWaves>(
            sc, sg, r0, begin, m, owned, flat, t, tsum, tflag, (MS_LDS float*)&slabs[0][0],
            (MS_LDS uint32_t*)wflag, wave, lane, mul, div);
        if (tn < ntiles) snext = find_seg(segs, nseg, begin + tn * kScanTile);
        __syncthreads();   // the staged tile and flags are rewritten by the next tile
        continue;
      }
      const char* src = static_cast<const char*>(sg.grad) + (r0 - sg.begin) * G::kBytes;
      uint32_t w[kPerLane][4];
#pragma unroll
      for (int k = 0; k < kPerLane; ++k)
        load_unit(src + ((wave * kPerLane + k) * 64 + lane) * 16, w[k]);
      if (tn < ntiles) snext = find_seg(segs, nseg, begin + tn * kScanTile);
      float g[kPerLane][kUnit];
#pragma unroll
      for (int k = 0; k < kPerLane; ++k) sc.template widen<false>(w[k], g[k]);
      MS_GLOBAL float* o = (MS_GLOBAL float*)flat + (r0 - begin);
      if constexpr (kUnit == 8) {
        // 2-byte gradients (units widen to 32 bytes): through the slab, so
        // that each of the wave's two stores writes one contiguous kilobyte
        // of whole lines; the slab keeps the values for the sum
        MS_LDS f4* slab = (MS_LDS f4*)slabs[wave];
        slab[2 * lane] = f4{g[0][0], g[0][1], g[0][2], g[0][3]};
        slab[2 * lane + 1] = f4{g[0][4], g[0][5], g[0][6], g[0][7]};
        __builtin_amdgcn_wave_barrier();
        const f4 x = slab[lane], y = slab[64 + lane];
        __builtin_amdgcn_wave_barrier();
        MS_GLOBAL f4* ow = (MS_GLOBAL f4*)(o + wave * 64 * kUnit);
        __builtin_nontemporal_store(x, ow + lane);
        __builtin_nontemporal_store(y, ow + 64 + lane);
      } else {
        // fp32 gradients: a unit is 16 bytes, lane l's units are already
        // contiguous across the wave
#pragma unroll
        for (int k = 0; k < kPerLane; ++k)
          __builtin_nontemporal_store(f4{g[k][0], g[k][1], g[k][2], g[k][3]},
                                      (MS_GLOBAL f4*)o + (wave * kPerLane + k) * 64 + lane);
        if (kStats) {
          slabs[wave][2 * lane] = f4{g[0][0], g[0][1], g[0][2], g[0][3]};
          slabs[wave][2 * lane + 1] = f4{g[1][0], g[1][1], g[1][2], g[1][3]};
        }
      }
      if constexpr (kStats) {
        const bool wb = __any((sc.packed & G::kTop) != 0);
        if (lane == 0) wflag[wave] = wb ? 1u : 0u;
        __syncthreads();
        if (wave == 0) {
          // lane l: its units l, l + 64, ... in increasing order, the order
          // of piece() (slab entry 2l + h: unit d*64 + l, its half h, for
          // 2-byte gradients; unit (2d + h)*64 + l for fp32)
          double acc = 0.0;
          if (owned) {
#pragma unroll
            for (int d = 0; d < kWaves; ++d) {
              const f4 lo = slabs[d][2 * lane], hi = slabs[d][2 * lane + 1];
              const float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
              for (int k = 0; k < 8; ++k) {
                const double x = static_cast<double>(v[k]);
                acc = __builtin_fma(x, x, acc);
              }
            }
          }
          const double tot = wave_sum(acc);
          if (lane == 0) {
            uint32_t f = 0;
#pragma unroll
            for (int d = 0; d < kWaves; ++d) f |= wflag[d];
            tsum[t] = tot;
            tflag[t] = f;
          }
        }
        __syncthreads();   // the slabs and flags are rewritten by the next tile
      }
    }
  }
}

// ------------------------------------------------------------------ K2
__global__ __launch_bounds__(kNormThreads) void k_norm_clip(
    const double* __restrict__ bsum, const uint32_t* __restrict__ bflag,
    int nblk, int ngroups, int has_clip, double max_norm, int scaler_enabled,
    double scale, int64_t good_steps, int64_t skipped_steps, int64_t window,
    double min_scale, double max_scale, ms_step_scalars_t* __restrict__ out,
    ms_step_scalars_t* __restrict__ out_host) {
  constexpr int kNormWaves = kNormThreads / 64;
  __shared__ double wsum[kNormWaves];
  __shared__ uint32_t wbad[kNormWaves];
  const int tid = threadIdx.x;
  float total = 0.0f;      // meaningful in thread 0
  uint32_t overflow = 0;   // meaningful in thread 0
  for (int gi = 0; gi < ngroups; ++gi) {
    const double* ps = bsum + static_cast<int64_t>(gi) * nblk;
    const uint32_t* pf = bflag + static_cast<int64_t>(gi) * nblk;
    double acc = 0.0;
    uint32_t bad = 0;
    if (nblk == kStatsBlocks) {
      // all of a thread's partials in flight at once, then added in the
      // same order as the loop below (slot tid, tid + kNormThreads, ...)
      constexpr int kPer = kStatsBlocks / kNormThreads;
      double x[kPer];
      uint32_t f[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        x[i] = ps[tid + i * kNormThreads];
        f[i] = pf[tid + i * kNormThreads];
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        acc += x[i];
        bad |= f[i];
      }
    } else {
      for (int b = tid; b < nblk; b += kNormThreads) {
        acc += ps[b];
        bad |= pf[b];
      }
    }
    const double w = wave_sum(acc);
    const bool wb = __any(bad != 0);
    if ((tid & 63) == 0) {
      wsum[tid >> 6] = w;
      wbad[tid >> 6] = wb ? 1u : 0u;
    }
    __syncthreads();
    if (tid == 0) {
      double gsum = 0.0;
      for (int k = 0; k < kNormWaves; ++k) {
        gsum += wsum[k];
        overflow |= wbad[k];
      }
      // per-group fp32 sum of squares, accumulated over groups in fp32
      total = total + static_cast<float>(gsum);
    }
    __syncthreads();
  }
  if (tid != 0) return;

  ms_step_scalars_t r;
  r.overflow = overflow ? 1u : 0u;
  r.ready = 0;
  r.sumsq = total;
  r.norm = sqrtf(total);
  r.clip_applied = 0;
  r.coef = 1.0f;
  r.coef64 = 1.0;
  double next_scale = scale;
  int64_t good = good_steps, skipped = skipped_steps;
  if (overflow) {
    if (scaler_enabled) {
      const double half = scale / 2.0;
      next_scale = half > min_scale ? half : min_scale;
      good = 0;
      skipped += 1;
    }
  } else {
    const double norm = static_cast<double>(r.norm);
    if (has_clip && norm > max_norm) {
      const double coef = max_norm / (norm + 1e-6);
      r.coef64 = coef;
      if (coef != 1.0) {
        r.clip_applied = 1;
        r.coef = static_cast<float>(coef);
      }
    }
    if (scaler_enabled) {
      good += 1;
      if (good >= window && scale < max_scale) {
        const double twice = scale * 2.0;
        next_scale = twice < max_scale ? twice : max_scale;
        good = 0;
      }
    }
  }
  r.next_scale = next_scale;
  r.next_good_steps = good;
  r.next_skipped_steps = skipped;
  *out = r;
  if (out_host) {
    // the host's copy, in pinned host memory: every field made visible
    // system-wide, then `ready` set, so a host that sees ready == 1 reads
    // the whole result (it may poll that word instead of waiting for the
    // kernel's completion)
    *out_host = r;
    __threadfence_system();
    *static_cast<volatile uint32_t*>(&out_host->ready) = 1u;
    __threadfence_system();
  }
}

// ------------------------------------------------------------------ K3
struct AdamScalars {
  float neg_lr, decay_alpha, beta1, omb1, beta2, omb2, bc1, bc2, eps,
      grad_scale, inv_scale;
  int decay, umode;
};

// One AdamW element, rounding exactly where minispeed's op sequence rounds
// (optim/adam.py:82-91 on top of flat.py:247 and flat.py:255-257):
//   g  = g / scale                      div_          (optional)
//   g  = g * coef                       mul_          (clip, optional)
//   p  = fma(p, -lr*wd, p)              add_(alpha)   (decay, optional)
//   m  = fma(g, 1-b1, m*b1)             mul_, add_(alpha)
//   v  = fma((1-b2)*g, g, v*b2)         mul_, addcmul_
//   d  = sqrt(v / bc2) + eps            div, sqrt, add_
//   p  = p + ((-lr) * (m / bc1)) / d    div, addcdiv_
__device__ inline void adamw1(float g, float& p, float& m, float& v,
                              const AdamScalars& h, bool clip, float coef) {
  if (clip) g = g * coef;
  if (h.decay) p = __builtin_fmaf(p, h.decay_alpha, p);
  m = __builtin_fmaf(g, h.omb1, m * h.beta1);
  v = __builtin_fmaf(h.omb2 * g, g, v * h.beta2);
  const float den = sqrtf(v / h.bc2) + h.eps;
  p = p + (h.neg_lr * (m / h.bc1)) / den;
}

// One block per kAdamTile-element tile (grid-stride when the grid is
// clamped), XCD-ordered.  A tile inside one segment takes the vector path:
// each lane streams kAdamUnroll quads in wave order, all loads of the tile
// first, then the arithmetic and all stores; the gradient and the model
// copy move as quads of their tile's kind (quad_kind), so a segment that
// starts off the quad alignment of the flat space stays on it.  Other tiles
// (segment edges, the tail, a 2-mod-4 gradient tile at either end of its
// segment) go element by element: lane j takes elements j, j +
// kAdamThreads, ...
template <class G, class M, bool kFlatGrad>
__global__ __launch_bounds__(kAdamThreads) void k_adamw(
    float* __restrict__ master, float* __restrict__ exp_avg,
    float* __restrict__ exp_avg_sq, const float* __restrict__ flat_grad,
    const ms_segment_t* __restrict__ segs, int nseg, int64_t begin,
    int64_t end, AdamScalars h, const ms_step_scalars_t* __restrict__ sc) {
  if (sc->overflow) return;   // skipped step: nothing is touched
  const bool clip = sc->clip_applied != 0;
  const float coef = sc->coef;
  const int lane = threadIdx.x;
  const int64_t n = end - begin;
  const int64_t ntiles = (n + kAdamTile - 1) / kAdamTile;
  const bool arrays_vec = aligned16(master) && aligned16(exp_avg) &&
                          aligned16(exp_avg_sq) &&
                          (!kFlatGrad || aligned16(flat_grad));
  __shared__ Kind2Lds<kAdamThreads> k2lds;
  int k2buf = 0;   // the buffer of the next kind-2 run

  for (int64_t t = xcd_tile(blockIdx.x, gridDim.x, kXcdChunk); t < ntiles; t += gridDim.x) {
    const int64_t t0 = begin + t * kAdamTile;
    const int64_t t1 = (t0 + kAdamTile < end) ? t0 + kAdamTile : end;
    const int s = find_seg(segs, nseg, t0);
    const ms_segment_t seg = segs[s];
    const int64_t so = t0 - seg.begin;   // the tile's offset in the segment
    // the gradient's and the model copy's quad kinds (every quad of a tile
    // has its tile's kind); a kind-2 gradient load reads one element before
    // and one after each quad, inside the segment only where the tile has
    // a neighbour on both sides
    const bool rg = !kFlatGrad && seg.grad != nullptr;
    const int gk = rg ? quad_kind(seg.grad, so, G::kBytes) : 0;
    const int mk = seg.model != nullptr ? quad_kind(seg.model, so, M::kBytes) : 0;
    const bool fast = t1 - t0 == kAdamTile && so >= 0 && t1 <= seg_end(seg) && arrays_vec &&
                      (gk != 2 || (so >= 1 && t1 < seg_end(seg)));
    if (fast) {
      const int64_t tl = t0 - begin;     // the tile's offset in the state arrays
      float g[kAdamUnroll][4], p[kAdamUnroll][4], m[kAdamUnroll][4], v[kAdamUnroll][4];
#pragma unroll
      for (int u = 0; u < kAdamUnroll; ++u) {
        const int64_t e = 4 * (static_cast<int64_t>(u) * kAdamThreads + lane);
        if (kFlatGrad) {
          ldq(flat_grad + tl + e, g[u]);
        } else if (rg) {
          ldq_any<G>(static_cast<const char*>(seg.grad) + (so + e) * G::kBytes, gk, g[u]);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) g[u][k] = 0.0f;
        }
        ldq(master + tl + e, p[u]);
        ldq(exp_avg + tl + e, m[u]);
        ldq(exp_avg_sq + tl + e, v[u]);
      }
#pragma unroll
      for (int u = 0; u < kAdamUnroll; ++u) {
        const int64_t e = 4 * (static_cast<int64_t>(u) * kAdamThreads + lane);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (!kFlatGrad && seg.grad) g[u][k] = unscale1(g[u][k], h.umode, h.grad_scale, h.inv_scale);
          adamw1(g[u][k], p[u][k], m[u][k], v[u][k], h, clip, coef);
        }
        stq(master + tl + e, p[u]);
        stq(exp_avg + tl + e, m[u]);
        stq(exp_avg_sq + tl + e, v[u]);
        if (seg.model) {
          char* q = static_cast<char*>(seg.model) + (so + e) * M::kBytes;
          if constexpr (M::kBytes == 2) {
            if (mk == 2) {
              stq_run_kind2<M, kAdamThreads>(q - 4 * lane * M::kBytes, lane, p[u],
                                             (MS_LDS uint32_t*)k2lds.w[k2buf]);
              k2buf ^= 1;
            } else {
              stq_any<M>(q, mk, p[u]);
            }
          } else {
            stq_any<M>(q, mk, p[u]);
          }
        }
      }
    } else {
      int sl = s;
      for (int k = 0; k < 4 * kAdamUnroll; ++k) {
        const int64_t i = t0 + lane + static_cast<int64_t>(k) * kAdamThreads;
        if (i >= t1) break;
        while (sl + 1 < nseg && i >= seg_end(segs[sl])) ++sl;
        const ms_segment_t& sg = segs[sl];
        const bool inside = i >= sg.begin && i < seg_end(sg);
        const int64_t l = i - begin;
        float g = 0.0f;
        if (kFlatGrad) {
          g = flat_grad[l];
        } else if (inside && sg.grad) {
          g = unscale1(G::widen(load_raw1<G>(sg.grad, i - sg.begin)), h.umode,
                       h.grad_scale, h.inv_scale);
        }
        float p = master[l], m = exp_avg[l], v = exp_avg_sq[l];
        adamw1(g, p, m, v, h, clip, coef);
        master[l] = p;
        exp_avg[l] = m;
        exp_avg_sq[l] = v;
        if (inside && sg.model) store_raw1<M>(sg.model, i - sg.begin, M::narrow(p));
      }
    }
  }
}

// ------------------------------------------------------------------ K4
// The tiling and vector / element paths of K3, with one read and one write
// stream.
template <class M>
__global__ __launch_bounds__(kStreamThreads) void k_cast(
    const float* __restrict__ flat, const ms_segment_t* __restrict__ segs,
    int nseg, int64_t begin, int64_t end) {
  const int lane = threadIdx.x;
  const int64_t n = end - begin;
  const int64_t ntiles = (n + kStreamTile - 1) / kStreamTile;
  const bool flat_vec = aligned16(flat);
  __shared__ Kind2Lds<kStreamThreads> k2lds;
  int k2buf = 0;   // the buffer of the next kind-2 run
  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    const int64_t t0 = begin + t * kStreamTile;
    const int64_t t1 = (t0 + kStreamTile < end) ? t0 + kStreamTile : end;
    const int s = find_seg(segs, nseg, t0);
    const ms_segment_t seg = segs[s];
    const int64_t so = t0 - seg.begin;
    const bool whole = t1 - t0 == kStreamTile && so >= 0 && t1 <= seg_end(seg) && flat_vec;
    const int64_t tl = t0 - begin;
    if (whole && quad_aligned(seg.model, so, M::kBytes)) {
      if (!seg.model) continue;
      float x[kStreamUnroll][4];
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u)
        ldq(flat + tl + 4 * (static_cast<int64_t>(u) * kStreamThreads + lane), x[u]);
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) {
        const int64_t e = 4 * (static_cast<int64_t>(u) * kStreamThreads + lane);
        stq_raw<M>(static_cast<char*>(seg.model) + (so + e) * M::kBytes, x[u]);
      }
    } else if (whole && seg.model) {
      // a model copy off the quads of the flat tiles (a segment shifted by
      // an earlier tensor of odd size, or a view at an odd offset): quads
      // of its kind; a separate branch, so that the aligned tiles above
      // keep their code (folding the kind into it cost the 8.03B cast 6%)
      const int mk = quad_kind(seg.model, so, M::kBytes);
      float x[kStreamUnroll][4];
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u)
        ldq(flat + tl + 4 * (static_cast<int64_t>(u) * kStreamThreads + lane), x[u]);
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) {
        const int64_t e = 4 * (static_cast<int64_t>(u) * kStreamThreads + lane);
        char* q = static_cast<char*>(seg.model) + (so + e) * M::kBytes;
        if constexpr (M::kBytes == 2) {
          if (mk == 2) {
            stq_run_kind2<M, kStreamThreads>(q - 4 * lane * M::kBytes, lane, x[u],
                                             (MS_LDS uint32_t*)k2lds.w[k2buf]);
            k2buf ^= 1;
          } else {
            stq_any<M>(q, mk, x[u]);
          }
        } else {
          stq_any<M>(q, mk, x[u]);
        }
      }
    } else {
      int sl = s;
      for (int k = 0; k < 4 * kStreamUnroll; ++k) {
        const int64_t i = t0 + lane + static_cast<int64_t>(k) * kStreamThreads;
        if (i >= t1) break;
        while (sl + 1 < nseg && i >= seg_end(segs[sl])) ++sl;
        const ms_segment_t& sg = segs[sl];
        if (i >= sg.begin && i < seg_end(sg) && sg.model)
          store_raw1<M>(sg.model, i - sg.begin, M::narrow(flat[i - begin]));
      }
    }
  }
}

// ------------------------------------------------------------------ K5
// dst[i] = (first ? 0 : dst[i]) + widen(src[i]) over the flat slices of up
// to kAccumRows gradients: one fp32 rounding per add, as torch's fp32 add_
// of a widened tensor.  The rows travel by value in the kernel arguments
// (about 3 KB), so a batch needs no table in device memory.  Block t works
// on tile t of the concatenated rows: row r owns tiles [tile0[r],
// tile0[r+1]), each of kStreamTile elements in wave order, with the
// non-temporal hint (the accumulation buffer and the gradient are each
// touched once per micro-batch); the slice and the gradient move as quads
// of their tile's kind (quad_kind).  The last partial tile of a row, and a
// 2-mod-4 gradient tile at either end of its row, step element by element.
// With statistics slots (ps / pf of the row) the block also writes the
// tile's fp64 sum of squares of the unscaled new values (each lane adds
// its own values in index order, waves reduce with a fixed xor tree, the
// wave sums are added in wave order: bitwise reproducible) and whether any
// new value is inf/nan.
constexpr int kAccumRows = MS_ACCUM_ROWS_PER_LAUNCH;
static_assert(kStreamTile == MS_ACCUM_TILE, "a K5 tile is one statistics slot");

struct AccumLaunch {
  int64_t tile0[kAccumRows + 1];   // tile0[nrows] = tiles of the launch
  float* dst[kAccumRows];
  const void* src[kAccumRows];
  int64_t numel[kAccumRows];
  double* ps[kAccumRows];          // per-tile sum of squares, or null
  uint32_t* pf[kAccumRows];        // per-tile inf/nan flag, or null
  uint64_t first;                  // bit r: row r overwrites dst
  int32_t nrows;
  int32_t umode;                   // unscale1 mode of the statistics
  float scale, inv;
};
static_assert(kAccumRows <= 64, "one bit of AccumLaunch::first per row");
static_assert(sizeof(AccumLaunch) <= 4096, "K5 rows must fit in the kernel arguments");
static_assert(sizeof(ms_accum_row_t) == 48, "ms_accum_row_t layout");

template <class D>
__global__ __launch_bounds__(kStreamThreads) void k_accumulate(const AccumLaunch L) {
  constexpr int kWaves = kStreamThreads / 64;
  __shared__ double wsum[kWaves];
  __shared__ uint32_t wbad[kWaves];
  const int lane = threadIdx.x;
  const int64_t ntiles = L.tile0[L.nrows];
  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    // the last row starting at or before t: rows with no tiles share their
    // tile0 with the next row, so this row holds t
    int lo = 0, hi = L.nrows - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (L.tile0[mid] <= t)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int r = lo;
    float* __restrict__ dst = L.dst[r];
    const char* __restrict__ src = static_cast<const char*>(L.src[r]);
    const int64_t n = L.numel[r];
    const bool first = ((L.first >> r) & 1u) != 0;
    const bool stats = L.ps[r] != nullptr;
    const int64_t tile = t - L.tile0[r];
    const int64_t e0 = tile * kStreamTile;
    const int64_t e1 = (e0 + kStreamTile < n) ? e0 + kStreamTile : n;
    double acc = 0.0;
    bool bad = false;
    auto count = [&](float x) {
      bad |= (__float_as_uint(x) & 0x7f800000u) == 0x7f800000u;
      const double d = static_cast<double>(unscale1(x, L.umode, L.scale, L.inv));
      acc = __builtin_fma(d, d, acc);
    };
    // quad kinds as in K3: the accumulation slice (fp32) and the gradient;
    // the tile's code is compiled twice, all-aligned quads and any kind, so
    // that the common tile runs no per-quad dispatch
    const int dk = quad_kind(dst, e0, 4), sk = quad_kind(src, e0, D::kBytes);
    auto quads = [&](auto aligned) {
      constexpr bool kAligned = decltype(aligned)::value;
      float g[kStreamUnroll][4], x[kStreamUnroll][4];
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) {
        const int64_t i = e0 + static_cast<int64_t>(u * kStreamThreads + lane) * 4;
        if constexpr (kAligned) {
          ldq_raw<D>(src + i * D::kBytes, g[u]);
          if (!first) ldq(dst + i, x[u]);
        } else {
          ldq_any<D>(src + i * D::kBytes, sk, g[u]);
          if (!first) ldq_any<DF32>(dst + i, dk, x[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) {
        const int64_t i = e0 + static_cast<int64_t>(u * kStreamThreads + lane) * 4;
#pragma unroll
        for (int k = 0; k < 4; ++k) x[u][k] = first ? g[u][k] : x[u][k] + g[u][k];
        if constexpr (kAligned)
          stq(dst + i, x[u]);
        else
          stq_any<DF32>(dst + i, dk, x[u]);
        if (stats) {
#pragma unroll
          for (int k = 0; k < 4; ++k) count(x[u][k]);
        }
      }
    };
    if (e1 - e0 == kStreamTile && (sk != 2 || (e0 >= 1 && e1 < n))) {
      if (dk == 0 && sk == 0)
        quads(BoolC<true>{});
      else
        quads(BoolC<false>{});
    } else {
      for (int64_t i = e0 + lane; i < e1; i += kStreamThreads) {
        const float g1 = D::widen(load_raw1<D>(src, i));
        const float x1 = first ? g1 : dst[i] + g1;
        dst[i] = x1;
        if (stats) count(x1);
      }
    }
    if (stats) {   // uniform over the block: one tile, one row
      const double w = wave_sum(acc);
      const bool wb = __any(bad);
      if ((lane & 63) == 0) {
        wsum[lane >> 6] = w;
        wbad[lane >> 6] = wb ? 1u : 0u;
      }
      __syncthreads();
      if (lane == 0) {
        double total = 0.0;
        uint32_t flag = 0;
#pragma unroll
        for (int k = 0; k < kWaves; ++k) {
          total += wsum[k];
          flag |= wbad[k];
        }
        L.ps[r][tile] = total;
        L.pf[r][tile] = flag;
      }
      __syncthreads();   // wsum / wbad are reused by the next tile
    }
  }
}

// ------------------------------------------------------------------ K2a
// Partial slot j covers tiles [j*ntiles/nblk, (j+1)*ntiles/nblk); lane l
// of the wave that folds it adds the tiles lo + l, lo + l + 64, ... in
// order, and the wave's fixed xor tree adds the lanes.  A fixed partition
// and order, so the result is a pure function of the tile statistics.  A
// wave folds kFoldSlots consecutive slots; when no slot holds more than 64
// tiles (every layout up to 2.1G flat indices per group) each lane has one
// tile per slot, and all of the wave's loads are issued before the sums.
constexpr int kFoldThreads = 256;
// (slots per wave at 124M params, K1 with the fold: 1 / 2 / 4 / 8 / 16:
// 55.0-55.3 / 54.4-55.3 / 54.9-56.3 / 57.4-58.5 / 61.3-61.7 us)
constexpr int kFoldSlots = 4;

__global__ __launch_bounds__(kFoldThreads) void k_fold_tiles(
    const double* __restrict__ ts, const uint32_t* __restrict__ tf, int64_t ntiles,
    double* __restrict__ bsum, uint32_t* __restrict__ bflag, int nblk) {
  const int lane = threadIdx.x & 63;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * (kFoldThreads / 64) + (threadIdx.x >> 6);
  const int64_t j0 = w * kFoldSlots;
  if (j0 >= nblk) return;   // whole waves
  double total[kFoldSlots];
  uint32_t flag[kFoldSlots];
  if ((ntiles + nblk - 1) / nblk <= 64) {
#pragma unroll
    for (int s = 0; s < kFoldSlots; ++s) {
      total[s] = 0.0;
      flag[s] = 0;
      const int64_t j = j0 + s;
      const int64_t k = j * ntiles / nblk + lane;
      if (j < nblk && k < (j + 1) * ntiles / nblk) {
        total[s] += ts[k];
        flag[s] = tf[k];
      }
    }
  } else {
    for (int s = 0; s < kFoldSlots; ++s) {
      total[s] = 0.0;
      flag[s] = 0;
      const int64_t j = j0 + s;
      if (j >= nblk) continue;
      const int64_t hi = (j + 1) * ntiles / nblk;
      for (int64_t k = j * ntiles / nblk + lane; k < hi; k += 64) {
        total[s] += ts[k];
        flag[s] |= tf[k];
      }
    }
  }
#pragma unroll
  for (int s = 0; s < kFoldSlots; ++s) {
    const double t = wave_sum(total[s]);
    const bool bad = __any(flag[s] != 0);
    if (lane == 0 && j0 + s < nblk) {
      bsum[j0 + s] = t;
      bflag[j0 + s] = bad ? 1u : 0u;
    }
  }
}

// ------------------------------------------------------------- launching
// Grid of a streaming kernel: one block per tile.  The kernels also walk
// their tiles grid-stride, so a clamped grid (more than 2^31 - 1 tiles)
// still covers every tile.
int stream_grid(int64_t ntiles) {
  int64_t g = ntiles;
  if (g > 0x7fffffff) g = 0x7fffffff;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MS_OK : static_cast<int>(e);
}

// How a kernel scales each widened gradient (see unscale1).  `unscale` is
// MS_SCALE_NONE, MS_SCALE_DIVIDE or MS_SCALE_MULTIPLY (checked by the caller).
int unscale_mode(int32_t unscale, float scale, float* inv) {
  *inv = 1.0f;
  if (unscale == MS_SCALE_NONE) return 0;
  if (unscale == MS_SCALE_MULTIPLY) return 3;
  int e = 0;
  const float mant = frexpf(scale, &e);   // scale = mant * 2^e
  if (mant == 0.5f && e - 1 <= 126 && e - 1 >= -126) {
    *inv = ldexpf(1.0f, 1 - e);
    return 1;
  }
  return 2;
}

bool valid_dtype(int32_t d) {
  return d == MS_DTYPE_F32 || d == MS_DTYPE_F16 || d == MS_DTYPE_BF16;
}

// K1's tiles over n flat indices
int64_t scan_tiles(int64_t n) { return (n + kScanTile - 1) / kScanTile; }

// Grid of K1 (kScanWaves tiles per block); the kernel walks its tiles
// grid-stride, so a clamped grid still covers every tile.
int scan_grid(int64_t ntiles, int tiles_per_block) {
  int64_t g = (ntiles + tiles_per_block - 1) / tiles_per_block;
  if (g > 0x7fffffff) g = 0x7fffffff;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

template <class G, int kScale>
void launch_stats_s(const ms_segment_t* segs, int nseg, int64_t begin, int64_t end, int64_t ob,
                    int64_t oe, float mul, float div, float* flat, double* tsum, uint32_t* tflag,
                    int64_t ntiles, hipStream_t st) {
  if (tsum) {
    if (flat) {
      hipLaunchKernelGGL((k_grad_stats<G, true, true, kScale>), dim3(scan_grid(ntiles, 1)),
                         dim3(64 * kScanWavesFlat), 0, st, segs, nseg, begin, end, ob, oe, mul,
                         div, flat, tsum, tflag, ntiles, 1, ntiles);
    } else {
      // runs of 2 and 4 tiles time alike over 60K-640K tiles, runs of 1 up
      // to 30% slower
      constexpr int kRun = MS_SCAN_RUN_READ;
      // the tiles holding the last kCacheKeepBytes of gradient
      const int64_t keep_tiles = kCacheKeepBytes / (int64_t(kScanTile) * G::kBytes);
      const int64_t keep_from = ntiles > keep_tiles ? ntiles - keep_tiles : 0;
      // the counted elements' flags from their sums wherever the scaling
      // cannot overflow a finite gradient (GradScan's kSumFlags)
      const bool sum_flags = kScale == kScaleNone ||
                             (kScale == kScaleMul && mul >= -1.0f && mul <= 1.0f) ||
                             (kScale == kScaleDiv && div >= 1.0f);
      auto go = [&](auto sf) {
        hipLaunchKernelGGL((k_grad_stats<G, false, true, kScale, decltype(sf)::value>),
                           dim3(scan_grid(ntiles, kScanWavesRead * kRun)),
                           dim3(64 * kScanWavesRead), 0, st, segs, nseg, begin, end, ob, oe, mul,
                           div, flat, tsum, tflag, ntiles, kRun, keep_from);
      };
      if (sum_flags)
        go(BoolC<true>{});
      else
        go(BoolC<false>{});
    }
  } else {
    hipLaunchKernelGGL((k_grad_stats<G, true, false, kScale>), dim3(scan_grid(ntiles, 1)),
                       dim3(64 * kScanWavesFlat), 0, st, segs, nseg, begin, end, ob, oe, mul, div,
                       flat, tsum, tflag, ntiles, 1, ntiles);
  }
}

template <class G>
void launch_stats(const ms_segment_t* segs, int nseg, int64_t begin,
                  int64_t end, int64_t ob, int64_t oe, int unscale, float scale,
                  float* flat, double* tsum, uint32_t* tflag, hipStream_t st) {
  const int64_t ntiles = scan_tiles(end - begin);
  if (ntiles == 0) return;
  float inv = 1.0f;
  switch (unscale_mode(unscale, scale, &inv)) {
    case 0:
      launch_stats_s<G, kScaleNone>(segs, nseg, begin, end, ob, oe, 1.0f, 1.0f, flat, tsum,
                                    tflag, ntiles, st);
      break;
    case 1:   // x / 2^k as x * 2^-k
      launch_stats_s<G, kScaleMul>(segs, nseg, begin, end, ob, oe, inv, 1.0f, flat, tsum, tflag,
                                   ntiles, st);
      break;
    case 3:   // x * factor
      launch_stats_s<G, kScaleMul>(segs, nseg, begin, end, ob, oe, scale, 1.0f, flat, tsum,
                                   tflag, ntiles, st);
      break;
    default:  // x / scale
      launch_stats_s<G, kScaleDiv>(segs, nseg, begin, end, ob, oe, 1.0f, scale, flat, tsum,
                                   tflag, ntiles, st);
      break;
  }
}

// K2a over ntiles tile slots into nblk partial slots (all written)
void launch_fold(const double* tsum, const uint32_t* tflag, int64_t ntiles, double* bsum,
                 uint32_t* bflag, int nblk, hipStream_t st) {
  constexpr int kSlotsPerBlock = kFoldThreads / 64 * kFoldSlots;
  const dim3 grid((nblk + kSlotsPerBlock - 1) / kSlotsPerBlock);
  hipLaunchKernelGGL(k_fold_tiles, grid, dim3(kFoldThreads), 0, st, tsum, tflag, ntiles, bsum,
                     bflag, nblk);
}

// Host-side checks of one K1 scan (ms_grad_stats' arguments); MS_OK or the
// error code, before anything is launched.
int check_scan(const ms_segment_t* segs, int32_t nseg, int32_t grad_dtype, int64_t begin,
               int64_t end, int32_t unscale, float grad_scale) {
  if (!valid_dtype(grad_dtype) || begin < 0 || end < begin) return MS_EINVAL;
  if (end > begin && (segs == nullptr || nseg <= 0)) return MS_ETABLE;
  if (nseg < 0 || nseg > kMaxSegs) return MS_ETABLE;
  if (unscale != MS_SCALE_NONE && unscale != MS_SCALE_DIVIDE && unscale != MS_SCALE_MULTIPLY)
    return MS_EINVAL;
  if (unscale == MS_SCALE_DIVIDE && !(grad_scale > 0.0f)) return MS_EINVAL;
  return MS_OK;
}

// K1 over [begin, end) (tile statistics into tsum / tflag when tsum is not
// NULL), then, with statistics, K2a folding them into bsum / bflag.
int launch_scan(const ms_segment_t* segs, int32_t nseg, int32_t grad_dtype, int64_t begin,
                int64_t end, int64_t own_begin, int64_t own_end, int32_t unscale,
                float grad_scale, float* flat_grad, double* tsum, uint32_t* tflag,
                double* bsum, uint32_t* bflag, int32_t nblk, hipStream_t st) {
  switch (grad_dtype) {
    case MS_DTYPE_F32:
      launch_stats<DF32>(segs, nseg, begin, end, own_begin, own_end, unscale, grad_scale,
                         flat_grad, tsum, tflag, st);
      break;
    case MS_DTYPE_F16:
      launch_stats<DF16>(segs, nseg, begin, end, own_begin, own_end, unscale, grad_scale,
                         flat_grad, tsum, tflag, st);
      break;
    default:
      launch_stats<DBF16>(segs, nseg, begin, end, own_begin, own_end, unscale, grad_scale,
                          flat_grad, tsum, tflag, st);
      break;
  }
  int rc = launch_status();
  if (rc != MS_OK || bsum == nullptr) return rc;
  launch_fold(tsum, tflag, scan_tiles(end - begin), bsum, bflag, nblk, st);
  return launch_status();
}

// Device address of `scratch` on the GPU that `st` belongs to (the current
// GPU for the null stream), looked up with that GPU current on the first
// call there and kept: every GPU holds its own copy of the array.
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
unsigned char* scratch_ptr[kMaxDevices] = {};

int scratch_base(hipStream_t st, unsigned char** out) {
  int dev = 0;
  hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return MS_EINVAL;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_ptr[dev] == nullptr) {
    int cur = 0;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return static_cast<int>(e);
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return static_cast<int>(e);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess) return static_cast<int>(e);
    if (p == nullptr) return MS_EINVAL;
    scratch_ptr[dev] = static_cast<unsigned char*>(p);
  }
  *out = scratch_ptr[dev];
  return MS_OK;
}

template <class G, class M>
void launch_adamw(float* p, float* m, float* v, const float* fg,
                  const ms_segment_t* segs, int nseg, int64_t begin, int64_t end,
                  const AdamScalars& h, const ms_step_scalars_t* sc,
                  hipStream_t st) {
  const int64_t ntiles = (end - begin + kAdamTile - 1) / kAdamTile;
  const dim3 grid(stream_grid(ntiles));
  const dim3 block(kAdamThreads);
  if (fg)
    hipLaunchKernelGGL((k_adamw<G, M, true>), grid, block, 0, st, p, m, v, fg,
                       segs, nseg, begin, end, h, sc);
  else
    hipLaunchKernelGGL((k_adamw<G, M, false>), grid, block, 0, st, p, m, v, fg,
                       segs, nseg, begin, end, h, sc);
}

template <class G>
void launch_adamw_m(int32_t model_dtype, float* p, float* m, float* v,
                    const float* fg, const ms_segment_t* segs, int nseg,
                    int64_t begin, int64_t end, const AdamScalars& h,
                    const ms_step_scalars_t* sc, hipStream_t st) {
  switch (model_dtype) {
    case MS_DTYPE_F32:
      launch_adamw<G, DF32>(p, m, v, fg, segs, nseg, begin, end, h, sc, st);
      break;
    case MS_DTYPE_F16:
      launch_adamw<G, DF16>(p, m, v, fg, segs, nseg, begin, end, h, sc, st);
      break;
    default:
      launch_adamw<G, DBF16>(p, m, v, fg, segs, nseg, begin, end, h, sc, st);
      break;
  }
}

}  // namespace

// =================================================================== C ABI
extern "C" {

int ms_abi_version(void) { return MS_ABI_VERSION; }

const char* ms_error_string(int code) {
  switch (code) {
    case MS_OK:
      return "success";
    case MS_EINVAL:
      return "invalid argument (size, range, dtype or required pointer)";
    case MS_ETABLE:
      return "segment count out of range";
    case MS_EBLOCKS:
      return "partial-sum workspace smaller than ms_stats_blocks(), or tile workspace "
             "smaller than ceil((end - begin) / MS_SCAN_TILE)";
    case MS_ESCRATCH:
      return "more groups than MS_SCRATCH_MAX_GROUPS, or a group of more than "
             "MS_SCRATCH_MAX_TILES tiles (the static scratch of ms_boundary_scalars_noalloc)";
    default:
      break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown error";
}

int ms_stats_blocks(void) { return kStatsBlocks; }

int ms_grad_stats(const ms_segment_t* segs, int32_t nseg, int32_t grad_dtype,
                  int64_t begin, int64_t end, int64_t own_begin,
                  int64_t own_end, int32_t unscale, float grad_scale,
                  float* flat_grad, double* tile_sumsq, uint32_t* tile_flag,
                  int64_t ntiles, double* block_sumsq, uint32_t* block_flag,
                  int32_t nblk, void* stream) {
  if (!valid_dtype(grad_dtype) || begin < 0 || end < begin) return MS_EINVAL;
  const bool stats = block_sumsq != nullptr;
  if (stats != (block_flag != nullptr) || stats != (tile_sumsq != nullptr) ||
      stats != (tile_flag != nullptr))
    return MS_EINVAL;
  if (!stats && flat_grad == nullptr) return MS_EINVAL;
  if (stats && (nblk < kStatsBlocks || ntiles < scan_tiles(end - begin))) return MS_EBLOCKS;
  const int rc = check_scan(segs, nseg, grad_dtype, begin, end, unscale, grad_scale);
  if (rc != MS_OK) return rc;
  if (!stats && end == begin) return MS_OK;
  return launch_scan(segs, nseg, grad_dtype, begin, end, own_begin, own_end, unscale,
                     grad_scale, flat_grad, tile_sumsq, tile_flag, block_sumsq, block_flag,
                     nblk, static_cast<hipStream_t>(stream));
}

int ms_boundary_scalars_noalloc(const ms_group_scan_t* groups, int32_t ngroups,
                                int32_t unscale, float grad_scale, int32_t has_clip,
                                double max_norm, int32_t scaler_enabled, double scale,
                                int64_t good_steps, int64_t skipped_steps, int64_t window,
                                double min_scale, double max_scale, ms_step_scalars_t* out,
                                ms_step_scalars_t* out_host, void* stream) {
  if (ngroups < 0 || (ngroups > 0 && groups == nullptr) || out == nullptr || window < 1)
    return MS_EINVAL;
  if (ngroups > MS_SCRATCH_MAX_GROUPS) return MS_ESCRATCH;
  for (int g = 0; g < ngroups; ++g) {
    const ms_group_scan_t& gs = groups[g];
    const int rc = check_scan(gs.segs, gs.nseg, gs.grad_dtype, gs.begin, gs.end, unscale,
                              grad_scale);
    if (rc != MS_OK) return rc;
    if (scan_tiles(gs.end - gs.begin) > MS_SCRATCH_MAX_TILES) return MS_ESCRATCH;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned char* base = nullptr;
  const int rc = scratch_base(st, &base);
  if (rc != MS_OK) return rc;
  constexpr size_t kSlots = static_cast<size_t>(MS_SCRATCH_MAX_GROUPS) * kStatsBlocks;
  double* sums = reinterpret_cast<double*>(base);
  uint32_t* flags = reinterpret_cast<uint32_t*>(base + sizeof(double) * kSlots);
  double* tsums = reinterpret_cast<double*>(base + (sizeof(double) + sizeof(uint32_t)) * kSlots);
  uint32_t* tflags = reinterpret_cast<uint32_t*>(
      reinterpret_cast<unsigned char*>(tsums) + sizeof(double) * MS_SCRATCH_MAX_TILES);
  for (int g = 0; g < ngroups; ++g) {
    const ms_group_scan_t& gs = groups[g];
    // K1 writes every tile slot of the group and the fold every one of its
    // kStatsBlocks partial slots, so the array needs no clearing between
    // calls; the next group's K1 reuses the tile slots after this fold
    // (same stream)
    const int lrc = launch_scan(gs.segs, gs.nseg, gs.grad_dtype, gs.begin, gs.end, gs.own_begin,
                                gs.own_end, unscale, grad_scale, nullptr, tsums, tflags,
                                sums + static_cast<int64_t>(g) * kStatsBlocks,
                                flags + static_cast<int64_t>(g) * kStatsBlocks, kStatsBlocks, st);
    if (lrc != MS_OK) return lrc;
  }
  hipLaunchKernelGGL(k_norm_clip, dim3(1), dim3(kNormThreads), 0, st, sums, flags, kStatsBlocks,
                     ngroups, has_clip, max_norm, scaler_enabled, scale, good_steps,
                     skipped_steps, window, min_scale, max_scale, out, out_host);
  return launch_status();
}

int ms_norm_clip(const double* block_sumsq, const uint32_t* block_flag,
                 int32_t nblk, int32_t ngroups, int32_t has_clip,
                 double max_norm, int32_t scaler_enabled, double scale,
                 int64_t good_steps, int64_t skipped_steps, int64_t window,
                 double min_scale, double max_scale, ms_step_scalars_t* out,
                 ms_step_scalars_t* out_host, void* stream) {
  if (!block_sumsq || !block_flag || !out || ngroups < 0) return MS_EINVAL;
  if (nblk < kStatsBlocks) return MS_EBLOCKS;
  if (window < 1) return MS_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_norm_clip, dim3(1), dim3(kNormThreads), 0, st, block_sumsq,
                     block_flag, nblk, ngroups, has_clip, max_norm,
                     scaler_enabled, scale, good_steps, skipped_steps, window,
                     min_scale, max_scale, out, out_host);
  return launch_status();
}

int ms_fused_adamw(float* master, float* exp_avg, float* exp_avg_sq,
                   const float* flat_grad, const ms_segment_t* segs,
                   int32_t nseg, int32_t grad_dtype, int32_t model_dtype,
                   int64_t begin, int64_t end, const ms_adamw_params_t* hp,
                   const ms_step_scalars_t* scalars, void* stream) {
  if (!valid_dtype(grad_dtype) || !valid_dtype(model_dtype)) return MS_EINVAL;
  if (!hp || !scalars || begin < 0 || end < begin) return MS_EINVAL;
  if (end == begin) return MS_OK;
  if (!master || !exp_avg || !exp_avg_sq) return MS_EINVAL;
  if (!segs || nseg <= 0 || nseg > kMaxSegs) return MS_ETABLE;
  if (hp->unscale != MS_SCALE_NONE && hp->unscale != MS_SCALE_DIVIDE) return MS_EINVAL;
  if (hp->unscale == MS_SCALE_DIVIDE && !(hp->grad_scale > 0.0f)) return MS_EINVAL;
  AdamScalars h;
  h.neg_lr = hp->neg_lr;
  h.decay_alpha = hp->decay_alpha;
  h.beta1 = hp->beta1;
  h.omb1 = hp->one_minus_beta1;
  h.beta2 = hp->beta2;
  h.omb2 = hp->one_minus_beta2;
  h.bc1 = hp->bias_c1;
  h.bc2 = hp->bias_c2;
  h.eps = hp->eps;
  h.grad_scale = hp->grad_scale;
  h.decay = hp->decay != 0;
  h.umode = unscale_mode(hp->unscale, hp->grad_scale, &h.inv_scale);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (grad_dtype) {
    case MS_DTYPE_F32:
      launch_adamw_m<DF32>(model_dtype, master, exp_avg, exp_avg_sq, flat_grad,
                           segs, nseg, begin, end, h, scalars, st);
      break;
    case MS_DTYPE_F16:
      launch_adamw_m<DF16>(model_dtype, master, exp_avg, exp_avg_sq, flat_grad,
                           segs, nseg, begin, end, h, scalars, st);
      break;
    default:
      launch_adamw_m<DBF16>(model_dtype, master, exp_avg, exp_avg_sq, flat_grad,
                            segs, nseg, begin, end, h, scalars, st);
      break;
  }
  return launch_status();
}

int ms_accumulate_grads(const ms_accum_row_t* rows, int32_t nrows, int32_t src_dtype,
                        int32_t unscale, float grad_scale, void* stream) {
  if (!valid_dtype(src_dtype) || nrows < 0 || (nrows > 0 && !rows)) return MS_EINVAL;
  if (unscale != MS_SCALE_NONE && unscale != MS_SCALE_DIVIDE) return MS_EINVAL;
  if (unscale == MS_SCALE_DIVIDE && !(grad_scale > 0.0f)) return MS_EINVAL;
  for (int32_t r = 0; r < nrows; ++r) {
    const ms_accum_row_t& row = rows[r];
    if (row.numel < 0 || (row.numel > 0 && (!row.dst || !row.src))) return MS_EINVAL;
    if ((row.tile_sumsq == nullptr) != (row.tile_flag == nullptr)) return MS_EINVAL;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  AccumLaunch L;
  float inv = 1.0f;
  L.umode = unscale_mode(unscale, grad_scale, &inv);
  L.scale = grad_scale;
  L.inv = inv;
  int32_t r = 0;
  while (r < nrows) {
    // the next launch: up to kAccumRows rows with elements
    L.nrows = 0;
    L.first = 0;
    int64_t tiles = 0;
    for (; r < nrows && L.nrows < kAccumRows; ++r) {
      const ms_accum_row_t& row = rows[r];
      if (row.numel == 0) continue;
      const int k = L.nrows++;
      L.tile0[k] = tiles;
      L.dst[k] = row.dst;
      L.src[k] = row.src;
      L.numel[k] = row.numel;
      L.ps[k] = row.tile_sumsq;
      L.pf[k] = row.tile_flag;
      if (row.first) L.first |= uint64_t(1) << k;
      tiles += (row.numel + kStreamTile - 1) / kStreamTile;
    }
    if (L.nrows == 0) break;
    L.tile0[L.nrows] = tiles;
    const dim3 grid(stream_grid(tiles));
    const dim3 block(kStreamThreads);
    switch (src_dtype) {
      case MS_DTYPE_F32:
        hipLaunchKernelGGL(k_accumulate<DF32>, grid, block, 0, st, L);
        break;
      case MS_DTYPE_F16:
        hipLaunchKernelGGL(k_accumulate<DF16>, grid, block, 0, st, L);
        break;
      default:
        hipLaunchKernelGGL(k_accumulate<DBF16>, grid, block, 0, st, L);
        break;
    }
    const int rc = launch_status();
    if (rc != MS_OK) return rc;
  }
  return MS_OK;
}

int ms_reduce_tile_stats(const double* tile_sumsq, const uint32_t* tile_flag, int64_t ntiles,
                         double* block_sumsq, uint32_t* block_flag, int32_t nblk,
                         void* stream) {
  if (ntiles < 0 || !block_sumsq || !block_flag) return MS_EINVAL;
  if (ntiles > 0 && (!tile_sumsq || !tile_flag)) return MS_EINVAL;
  if (nblk < kStatsBlocks) return MS_EBLOCKS;
  launch_fold(tile_sumsq, tile_flag, ntiles, block_sumsq, block_flag, nblk,
              static_cast<hipStream_t>(stream));
  return launch_status();
}

int ms_accumulate_grad(float* dst, const void* src, int32_t src_dtype, int64_t n,
                       int32_t first, void* stream) {
  if (!valid_dtype(src_dtype) || n < 0) return MS_EINVAL;
  if (n == 0) return MS_OK;
  if (!dst || !src) return MS_EINVAL;
  const ms_accum_row_t row{dst, src, n, first ? 1 : 0, 0, nullptr, nullptr};
  return ms_accumulate_grads(&row, 1, src_dtype, MS_SCALE_NONE, 1.0f, stream);
}

int ms_cast_to_model(const float* flat, int64_t begin, int64_t end,
                     const ms_segment_t* segs, int32_t nseg,
                     int32_t model_dtype, void* stream) {
  if (!valid_dtype(model_dtype) || begin < 0 || end < begin) return MS_EINVAL;
  if (end == begin) return MS_OK;
  if (!flat) return MS_EINVAL;
  if (!segs || nseg <= 0 || nseg > kMaxSegs) return MS_ETABLE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t ntiles = (end - begin + kStreamTile - 1) / kStreamTile;
  const dim3 grid(stream_grid(ntiles));
  const dim3 block(kStreamThreads);
  switch (model_dtype) {
    case MS_DTYPE_F32:
      hipLaunchKernelGGL(k_cast<DF32>, grid, block, 0, st, flat, segs, nseg,
                         begin, end);
      break;
    case MS_DTYPE_F16:
      hipLaunchKernelGGL(k_cast<DF16>, grid, block, 0, st, flat, segs, nseg,
                         begin, end);
      break;
    default:
      hipLaunchKernelGGL(k_cast<DBF16>, grid, block, 0, st, flat, segs, nseg,
                         begin, end);
      break;
  }
  return launch_status();
}

}  // extern "C"
