/* libaetherkv_probe.so: measurement utilities beside the product library, with no counterpart in
 * the reference.  bench.py times them next to the 4-bit D = 128 encode and the CSA decode step's
 * score pass as the practical streaming ceilings of those kernels' traffic.  Nothing in
 * libaetherkv.so uses them. */
#ifndef AETHERKV_PROBE_H_
#define AETHERKV_PROBE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { AEKV_PROBE_OK = 0, AEKV_PROBE_ERR_ARGS = 1, AEKV_PROBE_ERR_LAUNCH = 2 };

/* Moves the bytes of a 4-bit D = 128 bf16 encode of n_vec vectors (x [n_vec, 128] bf16 in; codes
 * [n_vec, 64] bytes and scale [n_vec] out) with the encode kernel's access pattern and non-temporal
 * stores but no transform (the outputs are xor folds of the inputs).  x and codes 16-byte aligned,
 * scale 4-byte aligned; a bad argument returns AEKV_PROBE_ERR_ARGS before anything is enqueued. */
int aekv_stream_probe(const void* x, int64_t n_vec, void* codes, float* scale, void* stream);

/* Moves the bytes of the CSA indexer's score pass over n_keys keys of one index cache (codes
 * [n_keys, row_bytes] with row_bytes 32 (4-bit) or 64 (8-bit), scale [n_keys] fp32), read in
 * groups of 128 keys per wave as the score kernel's decode groups; with keys set, it also writes 4
 * bytes per key to keys [n_keys] and 4 per 16 keys to smax [n_keys / 16], as the score kernel's
 * order keys and slot maxima (keys null: read only; smax must still be a writable word).  n_keys a
 * multiple of 128; codes 16-byte, scale and keys 8-byte, smax 4-byte aligned. */
int aekv_scan_probe(const void* codes, const float* scale, int64_t n_keys, int32_t row_bytes, void* keys,
                    uint32_t* smax, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* AETHERKV_PROBE_H_ */
