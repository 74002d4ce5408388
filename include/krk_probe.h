/*
 * krk_probe.h — the measurement probe bench.py times the GEMMs against
 * (libkrk_probe.so, built beside libkrk_gemm.so).  Not part of the GEMM's
 * C ABI and not on the decode path; no counterpart in the reference, whose
 * pickers time only the candidate GEMMs (engine/kernels/gemm.py:378-414).
 *
 * krk_probe_read — one launch that only reads `bytes` of device memory at
 * `p` (the pure-read floor of a projection's weight matrix): `blocks`
 * workgroups of 512 threads, 16-byte nontemporal loads, `unroll` (2, 4, 8
 * or 16) loads in flight per thread; `interleaved` 0: each workgroup streams
 * one contiguous chunk, 1: the workgroups take groups of unroll KB in turn.
 * `sink` is 1 KB of device memory the kernel may write (it keeps the loads
 * from being optimised away).  `bytes` a multiple of 16, `p` 16-byte
 * aligned, 1 <= blocks <= 65535.  Enqueues on `stream` and returns 0, -1 for
 * bad arguments (before any launch), -5 if the launch fails.
 */
#ifndef KRK_PROBE_H
#define KRK_PROBE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int krk_probe_read(const void* p, size_t bytes, void* sink, int blocks, int unroll, int interleaved, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KRK_PROBE_H */
