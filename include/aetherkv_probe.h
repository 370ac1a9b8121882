/* libaetherkv_probe.so: a measurement utility beside the product library, with no counterpart in
 * the reference.  bench.py times it next to the 4-bit D = 128 encode as the practical streaming
 * ceiling of that kernel's traffic.  Nothing in libaetherkv.so uses it. */
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

#ifdef __cplusplus
}
#endif
#endif /* AETHERKV_PROBE_H_ */
