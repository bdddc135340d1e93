/* CPython extension: packs the request-id dicts of the reference's
 * paged_attention signature (kernels/paged_attention.py:200-227) into the
 * int32 tables, lengths and shared-prefix statement the decode kernel takes,
 * in one pass over the dicts (the Python version spends most of its time
 * unboxing block ids one object at a time).
 *
 * pack(block_tables, seq_lens, block_size, num_blocks, out, width) -> mb
 * width(block_tables) -> the longest table's length
 *
 *   block_tables: dict request id -> sequence of block ids (insertion order)
 *   seq_lens:     dict request id -> length; a missing id means
 *                 len(blocks) * block_size
 *   out:          writable int32 buffer of at least n * (width + 2) entries,
 *                 width >= every table's length; receives [n][mb] tables
 *                 (unused cells 0), [n] lengths, [n] shared-prefix lengths
 *
 * Rules (the reference's, kernels/paged_attention.py:36-48):
 *   n_blocks = min(len(blocks), ceil(seq_len / block_size)); n_blocks <= 0
 *   raises RuntimeError; length = min(seq_len, n_blocks * block_size); a
 *   block id outside [-num_blocks, num_blocks) raises IndexError, negative
 *   ids count from the end.  Shared-prefix length of request b: leading
 *   equal ids of tables b - 1 and b, in tokens, cut to both lengths (0 for
 *   the first).
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* An int object's value: one-digit ints (|v| < 2**30, every block id in
 * practice) are read straight from the object on CPython < 3.12, whose int
 * layout this relies on; anything else goes through PyLong_AsLongLong. */
static inline long long id_value(PyObject* o) {
#if PY_VERSION_HEX < 0x030C0000
  if (PyLong_CheckExact(o)) {
    const Py_ssize_t sz = Py_SIZE(o);
    if (sz == 0) return 0;
    if (sz == 1) return (long long)((PyLongObject*)o)->ob_digit[0];
    if (sz == -1) return -(long long)((PyLongObject*)o)->ob_digit[0];
  }
#endif
  return PyLong_AsLongLong(o);
}

static long long floordiv(long long a, long long b) {
  long long q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}

static PyObject* pack(PyObject* self, PyObject* args) {
  (void)self;
  PyObject *tables, *lens_d;
  long long bs, nb, width;
  Py_buffer out;
  if (!PyArg_ParseTuple(args, "O!O!LLw*L", &PyDict_Type, &tables, &PyDict_Type, &lens_d, &bs, &nb, &out, &width))
    return NULL;
  PyObject* result = NULL;
  const Py_ssize_t n = PyDict_Size(tables);
  int32_t* o = (int32_t*)out.buf;
  long long* nblk = NULL;
  PyObject** seqs = NULL;
  if (bs <= 0 || nb <= 0 || width < 0) {
    PyErr_SetString(PyExc_ValueError, "block_size and num_blocks must be positive");
    goto done;
  }
  if ((long long)out.len < (long long)n * (width + 2) * (long long)sizeof(int32_t)) {
    PyErr_SetString(PyExc_ValueError, "output buffer too small");
    goto done;
  }
  nblk = (long long*)calloc(n > 0 ? n : 1, sizeof(long long));
  seqs = (PyObject**)calloc(n > 0 ? n : 1, sizeof(PyObject*));
  if (!nblk || !seqs) {
    PyErr_NoMemory();
    goto done;
  }
  int32_t* lens = o + n * width;  /* moved behind the compacted tables at the end */
  /* pass 1: lengths and block counts */
  Py_ssize_t pos = 0, i = 0;
  PyObject *key, *val;
  long long mb = 0;
  while (PyDict_Next(tables, &pos, &key, &val)) {
    PyObject* seq = PySequence_Fast(val, "block table must be a sequence");
    if (!seq) goto done;
    seqs[i] = seq;
    const long long len = PySequence_Fast_GET_SIZE(seq);
    long long seq_len;
    PyObject* sl = PyDict_GetItemWithError(lens_d, key);
    if (sl) {
      seq_len = PyLong_AsLongLong(sl);
      if (seq_len == -1 && PyErr_Occurred()) goto done;
    } else {
      if (PyErr_Occurred()) goto done;
      seq_len = len * bs;
    }
    long long want = floordiv(seq_len + bs - 1, bs);
    const long long nbk = len < want ? len : want;
    if (nbk <= 0) {
      PyErr_Format(PyExc_RuntimeError, "request %R: no KV blocks to attend (seq_len=%lld)", key, seq_len);
      goto done;
    }
    if (len > width) {
      PyErr_SetString(PyExc_ValueError, "width is smaller than a table");
      goto done;
    }
    nblk[i] = nbk;
    const long long cap_tokens = nbk * bs;
    lens[i] = (int32_t)(seq_len < cap_tokens ? seq_len : cap_tokens);
    if (nbk > mb) mb = nbk;
    ++i;
  }
  /* lengths to their final place [n * mb, n * mb + n) before the tables
     (rows of mb) are written over the front of the buffer */
  if (mb < width) memmove(o + n * mb, lens, (size_t)n * sizeof(int32_t));
  lens = o + n * mb;
  int32_t* shared = lens + n;
  /* pass 2: ids */
  pos = 0;
  i = 0;
  while (PyDict_Next(tables, &pos, &key, &val)) {
    PyObject** items = PySequence_Fast_ITEMS(seqs[i]);
    int32_t* row = o + i * mb;
    for (long long j = 0; j < nblk[i]; ++j) {
      long long bid = id_value(items[j]);
      if (bid == -1 && PyErr_Occurred()) goto done;
      if (bid < -nb || bid >= nb) {
        PyErr_Format(PyExc_IndexError, "request %R: block id %lld out of range for %lld cache blocks", key, bid, nb);
        goto done;
      }
      row[j] = (int32_t)(bid < 0 ? bid + nb : bid);
    }
    for (long long j = nblk[i]; j < mb; ++j) row[j] = 0;
    if (i == 0) {
      shared[0] = 0;
    } else {
      const int32_t* prev = o + (i - 1) * mb;
      const long long lim = nblk[i] < nblk[i - 1] ? nblk[i] : nblk[i - 1];
      long long k = 0;
      while (k < lim && prev[k] == row[k]) ++k;
      long long s = k * bs;
      if (lens[i - 1] < s) s = lens[i - 1];
      if (lens[i] < s) s = lens[i];
      shared[i] = (int32_t)(s > 0 ? s : 0);
    }
    ++i;
  }
  result = PyLong_FromLongLong(mb);
done:
  if (seqs) {
    for (Py_ssize_t k = 0; k < n; ++k) Py_XDECREF(seqs[k]);
    free(seqs);
  }
  free(nblk);
  PyBuffer_Release(&out);
  return result;
}

/* width(block_tables) -> the longest table's length (0 for no tables). */
static PyObject* width(PyObject* self, PyObject* arg) {
  (void)self;
  if (!PyDict_Check(arg)) {
    PyErr_SetString(PyExc_TypeError, "block_tables must be a dict");
    return NULL;
  }
  Py_ssize_t pos = 0, w = 0;
  PyObject *key, *val;
  while (PyDict_Next(arg, &pos, &key, &val)) {
    const Py_ssize_t n = PyObject_Length(val);
    if (n < 0) return NULL;
    if (n > w) w = n;
  }
  return PyLong_FromSsize_t(w);
}

static PyMethodDef methods[] = {
    {"pack", pack, METH_VARARGS, "pack(block_tables, seq_lens, block_size, num_blocks, out, width) -> mb"},
    {"width", width, METH_O, "width(block_tables) -> longest table length"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_tablepack", NULL, -1, methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__tablepack(void) { return PyModule_Create(&module); }
