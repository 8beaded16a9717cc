/* moe_diag.h — the bench's measurement probes (libmoe_diag.so, built from
 * moe_amd/diag/diag.hip beside the layer library).  Not part of the layer
 * ABI in include/moe_hip.h: they measure the machine the layer runs on.
 * Return codes are the MOE_* status codes; moe_diag_last_error() holds the
 * message of the last failure on the calling thread. */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char *moe_diag_last_error(void);

/* one cooperative launch of `blocks` blocks of 512 threads
 * (all resident: more is MOE_EINVAL) that pass `barriers` grid-wide
 * barriers (a device atomic per block on a counter, a polled generation
 * word; each poll bounded, state[2] set if a bound was hit).  `state`:
 * device u32[4], zero before the first call, left consistent for the next.
 * No counterpart in the reference. */
int moe_debug_grid_barrier(int32_t blocks, int32_t barriers, uint32_t *state, void *stream);

/* the issue rate of the two-pass MFMA kernels' instruction
 * mix.  `blocks` blocks of 256 * waves_per_simd (1 or 2) threads; each wave
 * runs `iters` iterations of `mfmas` V_MFMA_F32_32X32X16_F16 (two
 * independent chains) and `valus` f32 fmas on registers of their own, the
 * fmas after the MFMAs (interleave 0) or spread between them (1); one
 * float per thread into out[blocks * 256 * waves_per_simd].  Supported
 * (mfmas, valus, interleave): (8,0,0), (0,56,0), (8,56,0), (8,56,1),
 * (8,32,1).  No counterpart in the reference. */
int moe_debug_mfma_valu(int32_t mfmas, int32_t valus, int32_t interleave, int32_t waves_per_simd, int32_t blocks,
                        int32_t iters, float *out, void *stream);

/* read `bytes` (a multiple of 16, 16-byte aligned device
 * memory) once with a grid-stride 16-byte-load kernel of `blocks` blocks
 * (eight loads in flight per thread; nontemporal != 0: nontemporal loads),
 * writing one xor-fold per block to out[blocks]: the HBM read rate the
 * weight-streaming kernels are measured against.  No counterpart in the
 * reference. */
int moe_debug_stream_read(const void *src, uint64_t bytes, uint32_t *out, int32_t blocks, int32_t nontemporal,
                          void *stream);

#ifdef __cplusplus
}
#endif
