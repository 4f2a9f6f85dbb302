/*
 * minispeed_hbm_probe.h — C ABI of libms_hbm_probe.so, the streaming probes
 * behind bench.py's --hbm-ceilings mode.  Measurement only: minispeed has no
 * counterpart and nothing on the boundary path calls it.
 */
#ifndef MINISPEED_HBM_PROBE_H
#define MINISPEED_HBM_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSP_ABI_VERSION 2
#define MSP_MAX_ARRAYS 4

int msp_abi_version(void);

/*
 * One streaming pass over `nvec` 16-byte vectors of each array: rd[0..nread)
 * are read, wr[0..nwrite) are written (wr[k] == rd[k] makes array k an
 * in-place read-modify-write stream).  All arrays [dev] are 16-byte aligned
 * and hold nvec vectors.
 *   threads  : 64..1024, a multiple of 64
 *   unroll   : 1, 2, 4 or 8 vectors per lane per tile
 *   wave     : 0 = lane j owns `unroll` consecutive vectors of its tile;
 *              1 = load u of lane j is vector u*threads + j
 *   grid     : 0 = one block per tile; > 0 = that many blocks walking the
 *              tiles grid-stride
 *   nt_load / nt_store : non-temporal hints on the loads / stores
 *   sink [dev, >= 1024 words]: required when nwrite == 0; never written in
 *              practice (it keeps the loads of a read-only pass alive)
 * Returns 0, -1 for a bad argument (nothing launched), or a hipError_t.
 */
int msp_stream(const void* const* rd, int32_t nread, void* const* wr, int32_t nwrite,
               int64_t nvec, int32_t threads, int32_t unroll, int32_t wave, int32_t grid,
               int32_t nt_load, int32_t nt_store, uint32_t* sink, void* stream);

/*
 * K3's access pattern on a chosen layout of the AdamW state: per element
 * read g (fp16), p, m, v (fp32), update them with AdamW arithmetic, write
 * p, m, v and an fp16 copy; one 128-thread block per 512 elements, one
 * quad per lane, non-temporal hints on every stream.
 *   state[0..2] [dev] : p, m, v (interleave 0), or state[0] alone holding
 *                       [tile of T][p T | m T | v T] (interleave T)
 *   g, copy [dev]     : n fp16 elements each
 *   n                 : elements, a multiple of 512 and of T
 *   interleave        : 0, or T in {512, 1024, 2048, 4096}
 *   xcd_chunk         : 0 = block b on tile b; c > 0 = the 8 XCDs (blocks
 *                       dealt in turn) each take c consecutive tiles of
 *                       every group of 8c
 * Returns 0, -1 for a bad argument (nothing launched), or a hipError_t.
 */
int msp_adam_layout(float* const* state, const void* g, void* copy, int64_t n,
                    int32_t interleave, int32_t xcd_chunk, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MINISPEED_HBM_PROBE_H */
