/* Measurement entries of libfq_probe.so, the benchmark's probe library (not
 * part of the product library libfq_hip.so or its public header).  Both read
 * device memory the way a decode step does and compute nothing; bench.py
 * times them beside the decode to show the memory system's ceiling. */
#pragma once
#include "fq_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Measurement only; no counterpart in the reference.  Reads exactly what
 * fq_quest_decode_int4's single launch reads for the selection `mask`
 * (L, B, H_q, P) -- every page's K scale / min, then the K and V codes, V
 * scale / min and K scale / min of each KV group's union of selected pages --
 * with the same per-workgroup order and granularity, and computes nothing:
 * the memory system's ceiling for the step's access pattern.  `sink` is a
 * device word written only if the folded bytes hit an unlikely constant.
 * Workspace as fq_workspace_bytes (the union lists). */
int fq_read_decode_pages(const fq_int4_cache* cache, const uint8_t* mask, const int64_t mask_strides[4],
                         int32_t H_q, uint32_t* sink, void* workspace, size_t workspace_bytes, fq_stream_t stream);

/* Measurement only; no counterpart in the reference.  Reads `bytes` (a
 * nonzero multiple of 16) of one contiguous, 16-byte aligned device buffer
 * with plain streaming loads and computes nothing: the rate HBM gives a read
 * of that size with no access pattern, the reference point for
 * fq_read_decode_pages.  `sink` as there. */
int fq_read_stream(const void* buf, size_t bytes, uint32_t* sink, fq_stream_t stream);

#ifdef __cplusplus
}
#endif
