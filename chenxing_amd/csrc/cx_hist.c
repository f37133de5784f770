/* cx_hist.c -- CPython extension: the penalty windows of a batch, from the
 * caller's Python lists of token ids into the int32 [B, H] history array
 * the sampler library takes.
 *
 * The reference's callers hold histories as lists of Python ints
 * (chenxing/core/sampler.py:108, generated_ids: list[int]); unboxing them
 * one by one through numpy costs ~16 ns an id, which for a batch of 256
 * rows of 2048 ids is longer than the copy and both launches together.
 * This loop reads each list item's digits directly and applies
 * the reference's range rule on the way (sampler.py:68: ids outside
 * [0, vlim) are dropped, written here as -1).
 *
 * fill(seqs, rows, hist, hist_len, vlim) -> list of rows not filled
 *   seqs      list of lists (or tuples) of ids, one per entry of rows
 *   rows      list of row indices into hist
 *   hist      writable C-contiguous int32 buffer [B, H]
 *   hist_len  writable int32 buffer [B]
 *   vlim      ids in [0, vlim) are kept
 * A row is left to the caller (returned) when one of its items is not an
 * exact int, does not fit 64 bits, or the row is longer than H; nothing of
 * such a row is trusted, the caller rewrites it whole.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#if PY_VERSION_HEX < 0x030C0000
#include <longintrepr.h>
#endif

/* An exact int's value: 1 when it fits 64 bits.  Ints of up to two 30-bit
 * digits (every token id) are read from their digits directly on the
 * interpreters whose int layout is ob_size + digits (before 3.12); the rest
 * go through the C API. */
static inline int id_value(PyObject* it, long long* v) {
#if PY_VERSION_HEX < 0x030C0000
  const PyLongObject* L = (const PyLongObject*)it;
  const Py_ssize_t sz = Py_SIZE(L);
  if (sz >= -1 && sz <= 1) {
    *v = sz ? (sz > 0 ? (long long)L->ob_digit[0] : -(long long)L->ob_digit[0]) : 0;
    return 1;
  }
  if (sz == 2) {
    *v = (long long)L->ob_digit[0] | ((long long)L->ob_digit[1] << PyLong_SHIFT);
    return 1;
  }
#endif
  int ovf = 0;
  *v = PyLong_AsLongLongAndOverflow(it, &ovf);
  return !ovf;
}

static PyObject* fill(PyObject* self, PyObject* args) {
  PyObject *seqs, *rows, *hist_obj, *len_obj;
  long long vlim;
  (void)self;
  if (!PyArg_ParseTuple(args, "O!O!OOL", &PyList_Type, &seqs, &PyList_Type, &rows, &hist_obj,
                        &len_obj, &vlim))
    return NULL;
  const Py_ssize_t n = PyList_GET_SIZE(seqs);
  if (PyList_GET_SIZE(rows) != n) {
    PyErr_SetString(PyExc_ValueError, "seqs and rows differ in length");
    return NULL;
  }
  Py_buffer hb, lb;
  if (PyObject_GetBuffer(hist_obj, &hb, PyBUF_C_CONTIGUOUS | PyBUF_WRITABLE | PyBUF_FORMAT) < 0)
    return NULL;
  if (PyObject_GetBuffer(len_obj, &lb, PyBUF_C_CONTIGUOUS | PyBUF_WRITABLE | PyBUF_FORMAT) < 0) {
    PyBuffer_Release(&hb);
    return NULL;
  }
  PyObject* left = NULL;
  if (hb.ndim != 2 || hb.itemsize != 4 || lb.ndim != 1 || lb.itemsize != 4 ||
      lb.shape[0] != hb.shape[0]) {
    PyErr_SetString(PyExc_ValueError, "hist must be int32 [B, H] and hist_len int32 [B]");
    goto done;
  }
  const Py_ssize_t B = hb.shape[0], H = hb.shape[1];
  int32_t* hist = (int32_t*)hb.buf;
  int32_t* hlen = (int32_t*)lb.buf;
  left = PyList_New(0);
  if (!left) goto done;
  for (Py_ssize_t i = 0; i < n; ++i) {
    const Py_ssize_t b = PyLong_AsSsize_t(PyList_GET_ITEM(rows, i));
    if (b == -1 && PyErr_Occurred()) { Py_CLEAR(left); goto done; }
    if (b < 0 || b >= B) {
      PyErr_SetString(PyExc_IndexError, "row index out of range");
      Py_CLEAR(left);
      goto done;
    }
    PyObject* seq = PyList_GET_ITEM(seqs, i);
    PyObject** items;
    Py_ssize_t m;
    if (PyList_CheckExact(seq)) {
      items = PySequence_Fast_ITEMS(seq);
      m = PyList_GET_SIZE(seq);
    } else if (PyTuple_CheckExact(seq)) {
      items = PySequence_Fast_ITEMS(seq);
      m = PyTuple_GET_SIZE(seq);
    } else {
      m = -1;
      items = NULL;
    }
    int ok = m >= 0 && m <= H;
    int32_t* out = hist + b * H;
    for (Py_ssize_t j = 0; ok && j < m; ++j) {
      /* the int objects lie scattered over the heap: ask for later ones
         while this one is read */
      if (j + 16 < m) __builtin_prefetch(items[j + 16]);
      PyObject* it = items[j];
      long long v;
      if (!PyLong_CheckExact(it) || !id_value(it, &v)) { ok = 0; break; }
      out[j] = (v >= 0 && v < vlim) ? (int32_t)v : -1;
    }
    if (ok) {
      hlen[b] = (int32_t)m;
    } else if (PyList_Append(left, PyList_GET_ITEM(rows, i)) < 0) {
      Py_CLEAR(left);
      goto done;
    }
  }
done:
  PyBuffer_Release(&hb);
  PyBuffer_Release(&lb);
  return left;
}

static PyMethodDef methods[] = {
    {"fill", fill, METH_VARARGS, "Write the batch's penalty windows into hist / hist_len."},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef mod = {PyModuleDef_HEAD_INIT, "_cxhist",
                                 "Penalty windows from Python lists into int32 arrays.", -1,
                                 methods};

PyMODINIT_FUNC PyInit__cxhist(void) { return PyModule_Create(&mod); }
