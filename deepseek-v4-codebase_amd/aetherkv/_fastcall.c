/* Direct CPython calls of the libaetherkv C ABI entry points that callers make once per token.
 *
 * The reference's model calls tiled_prefill_attention once per target token (aether_2b/modeling.py:
 * 322,534) and its engine calls sparse_sink_attention / the decode step once per layer and token, so
 * the host cost of one call adds up.  ctypes converts each of these calls' 18-31 arguments through
 * per-argument converter objects (about 2 us per call); these METH_FASTCALL functions take the same
 * arguments as plain Python ints / floats / None (pointers as integers) and call the C ABI directly.
 * They add nothing: arguments, validation, status codes and messages are the library's own
 * (aetherkv._lib turns a nonzero status into the exception, as for the ctypes calls). */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

#include "aetherkv.h"

/* Python int (or None, for pointers) -> C value.  An overflow or a wrong type leaves a Python error
 * set, which the caller reports before calling into the library. */
static void* ptr_arg(PyObject* o) {
  if (o == Py_None) return NULL;
  return (void*)(uintptr_t)PyLong_AsUnsignedLongLongMask(o);
}
static int64_t i64_arg(PyObject* o) { return (int64_t)PyLong_AsLongLong(o); }
static int32_t i32_arg(PyObject* o) { return (int32_t)PyLong_AsLong(o); }
static float f32_arg(PyObject* o) { return (float)PyFloat_AsDouble(o); }

static int want_args(Py_ssize_t nargs, Py_ssize_t n, const char* who) {
  if (nargs == n) return 0;
  PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", who, n, nargs);
  return -1;
}

#define A(i) args[i]
#define RETURN_STATUS(call)                        \
  do {                                             \
    if (PyErr_Occurred()) return NULL;             \
    const int rc_ = (call);                        \
    return PyLong_FromLong(rc_);                   \
  } while (0)

/* aekv_sparse_sink_attention_ws(q, kv, idx, idx_dtype, sink, sink_numel, dtype, B, T, H, D, S, K,
 * scale, ws, ws_bytes, out, stream) */
static PyObject* f_sparse_sink_attention_ws(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (want_args(nargs, 18, "aekv_sparse_sink_attention_ws")) return NULL;
  void* q = ptr_arg(A(0));
  void* kv = ptr_arg(A(1));
  void* idx = ptr_arg(A(2));
  const int32_t idt = i32_arg(A(3));
  void* sink = ptr_arg(A(4));
  const int64_t sn = i64_arg(A(5));
  const int32_t dt = i32_arg(A(6));
  const int64_t B = i64_arg(A(7)), T = i64_arg(A(8)), H = i64_arg(A(9)), D = i64_arg(A(10));
  const int64_t S = i64_arg(A(11)), K = i64_arg(A(12));
  const float sc = f32_arg(A(13));
  void* ws = ptr_arg(A(14));
  const size_t wsb = (size_t)i64_arg(A(15));
  void* out = ptr_arg(A(16));
  void* st = ptr_arg(A(17));
  RETURN_STATUS(aekv_sparse_sink_attention_ws(q, kv, idx, idt, sink, sn, dt, B, T, H, D, S, K, sc, ws, wsb, out, st));
}

/* aekv_tiled_prefill_attention_ws(q, kv, sink, sink_numel, dtype, B, T, H, D, S, scale, tile_size,
 * ws, ws_bytes, out, stream) */
static PyObject* f_tiled_prefill_attention_ws(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (want_args(nargs, 16, "aekv_tiled_prefill_attention_ws")) return NULL;
  void* q = ptr_arg(A(0));
  void* kv = ptr_arg(A(1));
  void* sink = ptr_arg(A(2));
  const int64_t sn = i64_arg(A(3));
  const int32_t dt = i32_arg(A(4));
  const int64_t B = i64_arg(A(5)), T = i64_arg(A(6)), H = i64_arg(A(7)), D = i64_arg(A(8)), S = i64_arg(A(9));
  const float sc = f32_arg(A(10));
  const int32_t tile = i32_arg(A(11));
  void* ws = ptr_arg(A(12));
  const size_t wsb = (size_t)i64_arg(A(13));
  void* out = ptr_arg(A(14));
  void* st = ptr_arg(A(15));
  RETURN_STATUS(aekv_tiled_prefill_attention_ws(q, kv, sink, sn, dt, B, T, H, D, S, sc, tile, ws, wsb, out, st));
}

/* aekv_quant_sink_attention(q, codes, scale, sel, window, sink, diag, B, H, D, S, n_sel, W, bits,
 * scale, ws, ws_bytes, out, stream) */
static PyObject* f_quant_sink_attention(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (want_args(nargs, 19, "aekv_quant_sink_attention")) return NULL;
  void* q = ptr_arg(A(0));
  void* codes = ptr_arg(A(1));
  void* scale = ptr_arg(A(2));
  void* sel = ptr_arg(A(3));
  void* win = ptr_arg(A(4));
  void* sink = ptr_arg(A(5));
  void* diag = ptr_arg(A(6));
  const int64_t B = i64_arg(A(7)), H = i64_arg(A(8)), D = i64_arg(A(9)), S = i64_arg(A(10));
  const int64_t ns = i64_arg(A(11)), W = i64_arg(A(12));
  const int32_t bits = i32_arg(A(13));
  const float sm = f32_arg(A(14));
  void* ws = ptr_arg(A(15));
  const size_t wsb = (size_t)i64_arg(A(16));
  void* out = ptr_arg(A(17));
  void* st = ptr_arg(A(18));
  RETURN_STATUS(aekv_quant_sink_attention(q, codes, (const float*)scale, (const int64_t*)sel, win, (const float*)sink,
                                          (const float*)diag, B, H, D, S, ns, W, bits, sm, ws, wsb, out, st));
}

/* aekv_csa_decode_quant(index_q, index_weight, index_codes, index_scale, index_diag, valid, B, S, IH,
 * IC, index_bits, k, mode, q, kv_codes, kv_scale, window, sink, kv_diag, H, D, W, kv_bits, scale, ws,
 * ws_bytes, out_idx, out_score, out, stream) */
static PyObject* f_csa_decode_quant(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (want_args(nargs, 30, "aekv_csa_decode_quant")) return NULL;
  void* iq = ptr_arg(A(0));
  void* iw = ptr_arg(A(1));
  void* ic = ptr_arg(A(2));
  void* isc = ptr_arg(A(3));
  void* idg = ptr_arg(A(4));
  void* valid = ptr_arg(A(5));
  const int64_t B = i64_arg(A(6)), S = i64_arg(A(7));
  const int32_t IH = i32_arg(A(8)), IC = i32_arg(A(9)), ib = i32_arg(A(10)), k = i32_arg(A(11)), mode = i32_arg(A(12));
  void* q = ptr_arg(A(13));
  void* kc = ptr_arg(A(14));
  void* ksc = ptr_arg(A(15));
  void* win = ptr_arg(A(16));
  void* sink = ptr_arg(A(17));
  void* kdg = ptr_arg(A(18));
  const int64_t H = i64_arg(A(19)), D = i64_arg(A(20)), W = i64_arg(A(21));
  const int32_t kb = i32_arg(A(22));
  const float sm = f32_arg(A(23));
  void* ws = ptr_arg(A(24));
  const size_t wsb = (size_t)i64_arg(A(25));
  void* oi = ptr_arg(A(26));
  void* os = ptr_arg(A(27));
  void* out = ptr_arg(A(28));
  void* st = ptr_arg(A(29));
  RETURN_STATUS(aekv_csa_decode_quant((const float*)iq, (const float*)iw, ic, (const float*)isc, (const float*)idg,
                                      (const int32_t*)valid, B, S, IH, IC, ib, k, mode, q, kc, (const float*)ksc, win,
                                      (const float*)sink, (const float*)kdg, H, D, W, kb, sm, ws, wsb, (int64_t*)oi,
                                      (float*)os, out, st));
}

static PyMethodDef methods[] = {
    {"aekv_sparse_sink_attention_ws", (PyCFunction)(void (*)(void))f_sparse_sink_attention_ws, METH_FASTCALL, NULL},
    {"aekv_tiled_prefill_attention_ws", (PyCFunction)(void (*)(void))f_tiled_prefill_attention_ws, METH_FASTCALL, NULL},
    {"aekv_quant_sink_attention", (PyCFunction)(void (*)(void))f_quant_sink_attention, METH_FASTCALL, NULL},
    {"aekv_csa_decode_quant", (PyCFunction)(void (*)(void))f_csa_decode_quant, METH_FASTCALL, NULL},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_fastcall", NULL, -1, methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__fastcall(void) { return PyModule_Create(&module); }
