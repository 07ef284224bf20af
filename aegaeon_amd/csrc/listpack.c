/* Host-side packing of the reference's per-step request lists into the flat
 * arrays aegkv_prepare_inputs uploads (the lists Worker._prepare_model_inputs
 * walks, aegaeon/aegaeon/worker.py:596-646: RequestMeta tuples
 * (request_id, tokens, seq_len, context_len), aegaeon/aegaeon/request.py:96-102,
 * and one block table per request).  Python's iteration over those lists
 * costs ~30 ns per element; reading them through the CPython API costs a few.
 *
 *   pack_tables(tables) -> (ids: bytearray of int32, offsets: bytearray of int64)
 *       request b's table is ids[offsets[b]:offsets[b + 1]]
 *   pack_requests(requests) -> (seq_lens: bytearray of int32,
 *                               context_lens: bytearray of int32,
 *                               tokens: bytearray of int64)
 *       the new tokens of every request, in order; a request whose token list
 *       does not hold seq_len - context_len tokens raises ValueError
 *
 * Both accept lists or tuples (any sequence) of Python ints and raise
 * TypeError / OverflowError for anything else. */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <stdint.h>
#include <string.h>

static int long_in_range(PyObject* o, long long lo, long long hi, long long* out) {
  const long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) return -1;
  if (v < lo || v > hi) {
    PyErr_SetString(PyExc_OverflowError, "value out of range for its packed type");
    return -1;
  }
  *out = v;
  return 0;
}

static PyObject* pack_tables(PyObject* self, PyObject* arg) {
  (void)self;
  PyObject* outer = PySequence_Fast(arg, "block tables must be a sequence");
  if (!outer) return NULL;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(outer);
  PyObject** rows = PySequence_Fast_ITEMS(outer);
  PyObject* offsets = PyByteArray_FromStringAndSize(NULL, (n + 1) * (Py_ssize_t)sizeof(int64_t));
  PyObject* ids = NULL;
  PyObject** fast = NULL;
  if (!offsets) goto fail;
  fast = (PyObject**)PyMem_Calloc(n ? (size_t)n : 1, sizeof(PyObject*));
  if (!fast) {
    PyErr_NoMemory();
    goto fail;
  }
  int64_t* off = (int64_t*)PyByteArray_AS_STRING(offsets);
  off[0] = 0;
  for (Py_ssize_t b = 0; b < n; ++b) {
    fast[b] = PySequence_Fast(rows[b], "a block table must be a sequence");
    if (!fast[b]) goto fail;
    off[b + 1] = off[b] + PySequence_Fast_GET_SIZE(fast[b]);
  }
  ids = PyByteArray_FromStringAndSize(NULL, (Py_ssize_t)(off[n] * (int64_t)sizeof(int32_t)));
  if (!ids) goto fail;
  int32_t* dst = (int32_t*)PyByteArray_AS_STRING(ids);
  for (Py_ssize_t b = 0; b < n; ++b) {
    const Py_ssize_t m = PySequence_Fast_GET_SIZE(fast[b]);
    PyObject** items = PySequence_Fast_ITEMS(fast[b]);
    for (Py_ssize_t i = 0; i < m; ++i) {
      long long v;
      if (long_in_range(items[i], INT32_MIN, INT32_MAX, &v)) goto fail;
      *dst++ = (int32_t)v;
    }
  }
  for (Py_ssize_t b = 0; b < n; ++b) Py_DECREF(fast[b]);
  PyMem_Free(fast);
  Py_DECREF(outer);
  return Py_BuildValue("(NN)", ids, offsets);
fail:
  if (fast) {
    for (Py_ssize_t b = 0; b < n; ++b) Py_XDECREF(fast[b]);
    PyMem_Free(fast);
  }
  Py_XDECREF(ids);
  Py_XDECREF(offsets);
  Py_DECREF(outer);
  return NULL;
}

static PyObject* pack_requests(PyObject* self, PyObject* arg) {
  (void)self;
  PyObject* outer = PySequence_Fast(arg, "requests must be a sequence");
  if (!outer) return NULL;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(outer);
  PyObject** reqs = PySequence_Fast_ITEMS(outer);
  PyObject* seq = PyByteArray_FromStringAndSize(NULL, n * (Py_ssize_t)sizeof(int32_t));
  PyObject* ctx = PyByteArray_FromStringAndSize(NULL, n * (Py_ssize_t)sizeof(int32_t));
  PyObject* toks = NULL;
  PyObject** fast = NULL;
  if (!seq || !ctx) goto fail;
  fast = (PyObject**)PyMem_Calloc(n ? (size_t)n : 1, sizeof(PyObject*));
  if (!fast) {
    PyErr_NoMemory();
    goto fail;
  }
  int32_t* s = (int32_t*)PyByteArray_AS_STRING(seq);
  int32_t* c = (int32_t*)PyByteArray_AS_STRING(ctx);
  Py_ssize_t total = 0;
  for (Py_ssize_t b = 0; b < n; ++b) {
    PyObject* r = reqs[b];
    if (!PySequence_Check(r) || PySequence_Size(r) < 4) {
      PyErr_SetString(PyExc_TypeError,
                      "a request must be (request_id, tokens, seq_len, context_len)");
      goto fail;
    }
    PyObject* t = PySequence_GetItem(r, 1);
    PyObject* sl = PySequence_GetItem(r, 2);
    PyObject* cl = PySequence_GetItem(r, 3);
    long long sv = 0, cv = 0;
    const int bad = !t || !sl || !cl || long_in_range(sl, INT32_MIN, INT32_MAX, &sv) ||
                    long_in_range(cl, INT32_MIN, INT32_MAX, &cv);
    Py_XDECREF(sl);
    Py_XDECREF(cl);
    if (bad) {
      Py_XDECREF(t);
      goto fail;
    }
    fast[b] = PySequence_Fast(t, "a request's tokens must be a sequence");
    Py_DECREF(t);
    if (!fast[b]) goto fail;
    s[b] = (int32_t)sv;
    c[b] = (int32_t)cv;
    if ((long long)PySequence_Fast_GET_SIZE(fast[b]) != sv - cv) {
      PyErr_SetString(PyExc_ValueError,
                      "a request's tokens must be its seq_len - context_len new tokens");
      goto fail;
    }
    total += PySequence_Fast_GET_SIZE(fast[b]);
  }
  toks = PyByteArray_FromStringAndSize(NULL, total * (Py_ssize_t)sizeof(int64_t));
  if (!toks) goto fail;
  int64_t* dst = (int64_t*)PyByteArray_AS_STRING(toks);
  for (Py_ssize_t b = 0; b < n; ++b) {
    const Py_ssize_t m = PySequence_Fast_GET_SIZE(fast[b]);
    PyObject** items = PySequence_Fast_ITEMS(fast[b]);
    for (Py_ssize_t i = 0; i < m; ++i) {
      long long v;
      if (long_in_range(items[i], INT64_MIN, INT64_MAX, &v)) goto fail;
      *dst++ = (int64_t)v;
    }
  }
  for (Py_ssize_t b = 0; b < n; ++b) Py_DECREF(fast[b]);
  PyMem_Free(fast);
  Py_DECREF(outer);
  return Py_BuildValue("(NNN)", seq, ctx, toks);
fail:
  if (fast) {
    for (Py_ssize_t b = 0; b < n; ++b) Py_XDECREF(fast[b]);
    PyMem_Free(fast);
  }
  Py_XDECREF(seq);
  Py_XDECREF(ctx);
  Py_XDECREF(toks);
  Py_DECREF(outer);
  return NULL;
}

static PyMethodDef methods[] = {
    {"pack_tables", pack_tables, METH_O,
     "pack_tables(tables) -> (int32 ids bytearray, int64 offsets bytearray)"},
    {"pack_requests", pack_requests, METH_O,
     "pack_requests(requests) -> (int32 seq_lens, int32 context_lens, int64 tokens) bytearrays"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_listpack",
                                    "Packing of the per-step request lists", -1, methods,
                                    NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__listpack(void) { return PyModule_Create(&module); }
