/*
 * kraken_hip_diag.h -- measurement aids of the MI355X backend, in their own
 * library (kraken-infer_amd/build/libkraken_hip_diag.so, linked against
 * libkraken_hip.so).  Not part of the drop-in boundary: no counterpart in the
 * reference.  They give the benchmark the rates this GPU reaches, next to the
 * published peaks:
 *
 *  - kraken_hip_diag_stream_read reads `bytes` (a positive multiple of 16; source
 *    16-byte aligned) with nontemporal 16-byte loads from 256 x 256 threads and
 *    writes one float per thread (65,536 floats) to `sink`.
 *  - kraken_hip_diag_mfma_f16 runs `workgroups` workgroups of four waves, each wave
 *    issuing `iterations` x 8 v_mfma_f32_32x32x16_f16 (32,768 flops each), and writes
 *    `workgroups` x 256 floats to `sink`.
 *  - kraken_hip_diag_mfma_f16_denormals records what the f16 matrix cores do with
 *    an f16 denormal operand: v_mfma_f32_16x16x32_f16 and v_mfma_f32_16x16x16_f16
 *    with one element x in A (then in B) against ones, for x = 2^-15 and 2^-24
 *    (denormal) and 2^-14 (smallest normal).  It writes 12 floats, sink[4 v + 2 i
 *    + o] for value v, instruction i (0: 16x16x32, 1: 16x16x16) and operand o
 *    (0: A, 1: B): x where the operand survives, 0 where it is flushed.
 *
 * Status codes and argument checks follow kraken_hip.h; the message of the last
 * non-OK call on this thread is kraken_hip_diag_last_error().  The probes only
 * enqueue on the context's stream (they never wait; a host copy or
 * commit_graph on the context waits for them).
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
KRAKEN_API int kraken_hip_diag_mfma_f16_denormals(kraken_hip_context* context,
                                                  kraken_buffer sink);
KRAKEN_API const char* kraken_hip_diag_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
