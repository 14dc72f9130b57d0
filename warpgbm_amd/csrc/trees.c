/* Tree dicts of heap-ordered tree records (CPython extension
 * warpgbm_amd._trees).
 *
 * A fit hands back every tree as a nested dict in the reference's format
 * (warpgbm/core.py:653-658: {"feature", "bin", "left", "right"} for a split,
 * {"leaf_value", "samples"} for a leaf).  The engine writes trees as heap
 * records (node h has children 2h+1 and 2h+2; feature >= 0 a split, -1 a
 * leaf, -2 no node), and building the dicts is the fit's largest host cost.
 * Done here in C (about a third of the time of the same loop in Python), it
 * fits into the launching thread's slack while later rounds run on the GPU.
 *
 * heaps_to_dicts(feat, bin, leaf, count, H) -> list of len(feat) / H trees
 *   feat, bin: int32; leaf: float32; count: int64; C-contiguous buffers of
 *   the same length, a multiple of H.  A tree whose root is absent is None;
 *   an absent child of a split is None.  Values become Python ints and
 *   floats (float32 widened exactly), as numpy's tolist() gives them. */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <string.h>

static PyObject *k_feature, *k_bin, *k_left, *k_right, *k_leaf_value, *k_samples;

/* a dict sized for its keys up front (no growth while they are inserted) */
static inline PyObject* new_dict(Py_ssize_t n) {
#if PY_VERSION_HEX < 0x030D0000
  return _PyDict_NewPresized(n);
#else
  (void)n;
  return PyDict_New();
#endif
}

static int get_buf(PyObject* o, Py_buffer* b, Py_ssize_t itemsize, const char* kinds,
                   const char* what) {
  if (PyObject_GetBuffer(o, b, PyBUF_C_CONTIGUOUS | PyBUF_FORMAT) < 0) return -1;
  const char* f = b->format ? b->format : "B";
  if (*f == '<' || *f == '=' || *f == '@') ++f;
  if (b->itemsize != itemsize || f[0] == '\0' || f[1] != '\0' || !strchr(kinds, f[0])) {
    PyErr_Format(PyExc_TypeError, "%s: expected %zd-byte items of kind '%s', got '%s'", what,
                 itemsize, kinds, b->format ? b->format : "B");
    PyBuffer_Release(b);
    return -1;
  }
  return 0;
}

static PyObject* heaps_to_dicts(PyObject* self, PyObject* args) {
  (void)self;
  PyObject *of, *ob, *ol, *oc;
  Py_ssize_t H;
  if (!PyArg_ParseTuple(args, "OOOOn", &of, &ob, &ol, &oc, &H)) return NULL;
  if (H < 1) return PyErr_Format(PyExc_ValueError, "H must be positive");
  Py_buffer bf, bb, bl, bc;
  if (get_buf(of, &bf, 4, "il", "feat") < 0) return NULL;
  if (get_buf(ob, &bb, 4, "il", "bin") < 0) goto fail_f;
  if (get_buf(ol, &bl, 4, "f", "leaf") < 0) goto fail_b;
  if (get_buf(oc, &bc, 8, "qlL", "count") < 0) goto fail_l;
  PyObject* out = NULL;
  PyObject** nodes = NULL;
  const Py_ssize_t n = bf.len / 4;
  if (bb.len / 4 != n || bl.len / 4 != n || bc.len / 8 != n || n % H != 0) {
    PyErr_SetString(PyExc_ValueError, "heaps_to_dicts: buffers of different lengths");
    goto done;
  }
  const int32_t* feat = (const int32_t*)bf.buf;
  const int32_t* bin = (const int32_t*)bb.buf;
  const float* leaf = (const float*)bl.buf;
  const int64_t* count = (const int64_t*)bc.buf;
  const Py_ssize_t M = n / H;
  nodes = (PyObject**)PyMem_Calloc((size_t)H, sizeof(PyObject*));
  out = PyList_New(M);
  if (!nodes || !out) {
    Py_CLEAR(out);
    PyErr_NoMemory();
    goto done;
  }
  for (Py_ssize_t t = 0; t < M; ++t) {
    const int32_t* f = feat + t * H;
    /* bottom-up: a node's children are built before it */
    for (Py_ssize_t h = H - 1; h >= 0; --h) {
      PyObject* d = NULL;
      if (f[h] >= 0) {
        const Py_ssize_t l = 2 * h + 1, r = 2 * h + 2;
        if (r >= H) {
          PyErr_Format(PyExc_ValueError, "tree %zd: split at heap node %zd has no child slots",
                       t, h);
          goto tree_fail;
        }
        d = new_dict(4);
        PyObject* fv = PyLong_FromLong(f[h]);
        PyObject* bv = PyLong_FromLong(bin[t * H + h]);
        PyObject* lv = nodes[l] ? nodes[l] : Py_None;
        PyObject* rv = nodes[r] ? nodes[r] : Py_None;
        if (!d || !fv || !bv || PyDict_SetItem(d, k_feature, fv) < 0 ||
            PyDict_SetItem(d, k_bin, bv) < 0 || PyDict_SetItem(d, k_left, lv) < 0 ||
            PyDict_SetItem(d, k_right, rv) < 0) {
          Py_XDECREF(fv);
          Py_XDECREF(bv);
          Py_XDECREF(d);
          goto tree_fail;
        }
        Py_DECREF(fv);
        Py_DECREF(bv);
        /* the children now live in d */
        Py_CLEAR(nodes[l]);
        Py_CLEAR(nodes[r]);
        /* A tree of dicts holds no reference cycle, so the cyclic collector
         * need not track it (leaf dicts, holding only numbers, are untracked
         * by CPython itself): a forest of 2000 trees is otherwise ~250k
         * containers that every full collection walks.  A container stored
         * into d later makes CPython track d again. */
        PyObject_GC_UnTrack(d);
      } else if (f[h] == -1) {
        d = new_dict(2);
        PyObject* vv = PyFloat_FromDouble((double)leaf[t * H + h]);
        PyObject* cv = PyLong_FromLongLong((long long)count[t * H + h]);
        if (!d || !vv || !cv || PyDict_SetItem(d, k_leaf_value, vv) < 0 ||
            PyDict_SetItem(d, k_samples, cv) < 0) {
          Py_XDECREF(vv);
          Py_XDECREF(cv);
          Py_XDECREF(d);
          goto tree_fail;
        }
        Py_DECREF(vv);
        Py_DECREF(cv);
      } else {
        continue; /* no node */
      }
      Py_XDECREF(nodes[h]);
      nodes[h] = d;
    }
    /* the root (or None); nodes below an absent parent are dropped */
    PyList_SET_ITEM(out, t, nodes[0] ? nodes[0] : (Py_INCREF(Py_None), Py_None));
    nodes[0] = NULL;
    for (Py_ssize_t h = 1; h < H; ++h) Py_CLEAR(nodes[h]);
    continue;
  tree_fail:
    for (Py_ssize_t h = 0; h < H; ++h) Py_CLEAR(nodes[h]);
    Py_CLEAR(out);
    goto done;
  }
done:
  PyMem_Free(nodes);
  PyBuffer_Release(&bc);
  PyBuffer_Release(&bl);
  PyBuffer_Release(&bb);
  PyBuffer_Release(&bf);
  return out;
fail_l:
  PyBuffer_Release(&bl);
fail_b:
  PyBuffer_Release(&bb);
fail_f:
  PyBuffer_Release(&bf);
  return NULL;
}

static PyMethodDef methods[] = {
    {"heaps_to_dicts", heaps_to_dicts, METH_VARARGS,
     "heaps_to_dicts(feat, bin, leaf, count, H) -> list of tree dicts"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_trees", NULL, -1, methods,
                                    NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__trees(void) {
  k_feature = PyUnicode_InternFromString("feature");
  k_bin = PyUnicode_InternFromString("bin");
  k_left = PyUnicode_InternFromString("left");
  k_right = PyUnicode_InternFromString("right");
  k_leaf_value = PyUnicode_InternFromString("leaf_value");
  k_samples = PyUnicode_InternFromString("samples");
  if (!k_feature || !k_bin || !k_left || !k_right || !k_leaf_value || !k_samples) return NULL;
  return PyModule_Create(&module);
}
