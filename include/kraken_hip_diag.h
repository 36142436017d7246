/*
 * kraken_hip_diag.h -- measurement aids of the MI355X backend.  Not part of the
 * drop-in boundary: no counterpart in the reference.  They give the benchmark
 * the rates this GPU reaches, next to the published peaks:
 *
 *  - kraken_hip_diag_stream_read reads `bytes` (a positive multiple of 16; source
 *    16-byte aligned) with nontemporal 16-byte loads from 256 x 256 threads and
 *    writes one float per thread (65,536 floats) to `sink`.
 *  - kraken_hip_diag_mfma_f16 runs `workgroups` workgroups of four waves, each wave
 *    issuing `iterations` x 8 v_mfma_f32_32x32x16_f16 (32,768 flops each), and writes
 *    `workgroups` x 256 floats to `sink`.
 *
 * Status codes, argument checks and synchronisation follow kraken_hip.h.
 */
#ifndef KRAKEN_HIP_DIAG_H
#define KRAKEN_HIP_DIAG_H

#include "kraken_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

KRAKEN_API int kraken_hip_diag_stream_read(kraken_hip_context* context, kraken_buffer source,
                                           size_t bytes, kraken_buffer sink);
KRAKEN_API int kraken_hip_diag_mfma_f16(kraken_hip_context* context, uint32_t workgroups,
                                        uint32_t iterations, kraken_buffer sink);

#ifdef __cplusplus
}
#endif

#endif
