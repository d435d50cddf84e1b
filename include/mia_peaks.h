/*
 * mia_peaks.h -- measured peaks of the MI355X roofs the attention kernels sit
 * under.  Part of libmiattn.so.
 *
 * No counterpart in the reference's FFI: these play the role of its peak
 * benchmark (inmem_peak.m:89-111, the ANE's measured throughput ceiling
 * reported beside its kernels), so that a kernel's fraction can be quoted
 * against the published peak and against what this part actually sustains.
 * Each call launches one kernel on `stream` (NULL: the library stream) and
 * returns at once; time a loop of calls with mia_event_record.
 * Errors return a mia_status; the message is in mia_last_error().
 */
#ifndef MIA_PEAKS_H
#define MIA_PEAKS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` (a positive multiple of 16) of device memory once: a plain
 * grid-stride stream, four 16-byte loads in flight per thread. */
int mia_peak_read_stream(const void *buf_dev, size_t bytes, void *stream);

/* Reads one layer's K and V window (L slots from ring slot `start`,
 * wrapping at max_seq; 1 <= L <= max_seq, 0 <= start < max_seq) in the
 * access pattern of the decode kernel of mia_decode_step, with the same
 * chunking, and no arithmetic: the HBM bound of that kernel's loads. */
int mia_peak_read_ring(const uint16_t *k_layer_dev, const uint16_t *v_layer_dev, int n_kv_heads,
                       int max_seq, int L, int start, void *stream);

/* `iters` rounds of four independent v_mfma_f32_32x32x16_f16 chains in two
 * waves per SIMD on every CU; *flop receives the launch's FLOP count
 * (32 x 32 x 16 x 2 per instruction). */
int mia_peak_mfma_f16(int iters, double *flop, void *stream);

/* One empty kernel of `workgroups` x `threads` (1..1024).  Under
 * mia_profile_begin its dispatch-stamped duration is recorded as profile
 * kind 4, measured as the attention kernels' durations are: what a kernel
 * with no body costs (grid dispatch, the cache maintenance at the kernel
 * boundaries, the completion signal) by that method. */
int mia_peak_empty(int workgroups, int threads, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MIA_PEAKS_H */
