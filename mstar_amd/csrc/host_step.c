/* Host bookkeeping of one planning step, as a CPython extension.
 *
 * The per-request loops of the GPU pack's host side -- the FIFO page need of
 * every request (mstar/engine/kv_store.py:463-482, alloc up to
 * seq_len + new tokens), handing out the pages in request order, the block
 * table delta (pages not yet on the device) and the per-request metadata the
 * pack kernel reads, and advance_seq_lens (mstar/engine/cache_manager.py:
 * 811-838) -- over the KVRequestState objects themselves.  The Python
 * versions of the same loops (kv_store.PagedAllocationManager.alloc_batch,
 * DeviceBlockTable.prepare_meta, BatchedCacheManager.advance_seq_lens) stay
 * as the specification; tests run both on the same state sequences.
 *
 * State attributes live in each instance's __dict__ (KVRequestState is a
 * plain dataclass) and are read and written there (CPython 3.10); an object
 * without a dict, or a later interpreter, uses generic attribute access.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static PyObject *k_seq_len, *k_pos, *k_pages, *k_slot, *k_dev_list, *k_dev_len, *k_dev_ends;

/* The instance dict is read directly on CPython 3.10 (the interpreter this
 * package builds for); later versions keep instance attributes in their own
 * layout, so there the generic attribute protocol is used. */
#ifndef MI_DIRECT_DICT /* -DMI_DIRECT_DICT=0 builds the generic branch on any version (tested that way) */
#if PY_VERSION_HEX < 0x030B0000
#define MI_DIRECT_DICT 1
#else
#define MI_DIRECT_DICT 0
#endif
#endif

/* Module name: _host_step, or another name given with -DMI_HOST_STEP_MODULE
 * (the generic-attribute test build is loaded beside the default one). */
#ifndef MI_HOST_STEP_MODULE
#define MI_HOST_STEP_MODULE _host_step
#endif
#define MI_STR_(x) #x
#define MI_STR(x) MI_STR_(x)
#define MI_CAT_(a, b) a##b
#define MI_CAT(a, b) MI_CAT_(a, b)

/* New reference to attribute `k` of `o`, or NULL with an exception set. */
static PyObject* get_attr(PyObject* o, PyObject* k) {
#if MI_DIRECT_DICT
  PyObject** dp = _PyObject_GetDictPtr(o);
  if (dp && *dp) {
    PyObject* v = PyDict_GetItemWithError(*dp, k);
    if (v) {
      Py_INCREF(v);
      return v;
    }
    if (PyErr_Occurred()) return NULL;
  }
#endif
  return PyObject_GetAttr(o, k);
}

static int set_attr(PyObject* o, PyObject* k, PyObject* v) {
#if MI_DIRECT_DICT
  PyObject** dp = _PyObject_GetDictPtr(o);
  if (dp && *dp) return PyDict_SetItem(*dp, k, v);
#endif
  return PyObject_SetAttr(o, k, v);
}

static int get_long(PyObject* o, PyObject* k, long* out) {
  PyObject* v = get_attr(o, k);
  if (!v) return -1;
  *out = PyLong_AsLong(v);
  Py_DECREF(v);
  return (*out == -1 && PyErr_Occurred()) ? -1 : 0;
}

static int set_long(PyObject* o, PyObject* k, long x) {
  PyObject* v = PyLong_FromLong(x);
  if (!v) return -1;
  const int r = set_attr(o, k, v);
  Py_DECREF(v);
  return r;
}

/* seq_lens[i] (a sequence of ints), or 1 when seq_lens is None. */
static int seq_item(PyObject* fast, Py_ssize_t i, long* out) {
  if (!fast) {
    *out = 1;
    return 0;
  }
  *out = PyLong_AsLong(PySequence_Fast_GET_ITEM(fast, i));
  return (*out == -1 && PyErr_Occurred()) ? -1 : 0;
}

/* needs(states, seq_lens, page_size) -> (total, bytearray of int32 need[n])
 * need[i] = max(0, ceil((seq_len + seq_lens[i]) / page_size) - len(page_indices)). */
static PyObject* py_needs(PyObject* self, PyObject* args) {
  PyObject *states, *seq_lens;
  long ps;
  if (!PyArg_ParseTuple(args, "OOl", &states, &seq_lens, &ps)) return NULL;
  if (ps <= 0) return PyErr_Format(PyExc_ValueError, "page_size must be positive");
  PyObject* sf = PySequence_Fast(states, "states must be a sequence");
  if (!sf) return NULL;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(sf);
  PyObject* lf = NULL;
  if (seq_lens != Py_None) {
    lf = PySequence_Fast(seq_lens, "seq_lens must be a sequence");
    if (!lf) goto fail;
    if (PySequence_Fast_GET_SIZE(lf) != n) {
      PyErr_Format(PyExc_ValueError, "%zd seq_lens for %zd states", PySequence_Fast_GET_SIZE(lf), n);
      goto fail;
    }
  }
  PyObject* out = PyByteArray_FromStringAndSize(NULL, (Py_ssize_t)(4 * n));
  if (!out) goto fail;
  int32_t* need = (int32_t*)PyByteArray_AS_STRING(out);
  long long total = 0;
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* st = PySequence_Fast_GET_ITEM(sf, i);
    long seq, sl;
    if (get_long(st, k_seq_len, &seq) || seq_item(lf, i, &sl)) {
      Py_DECREF(out);
      goto fail;
    }
    PyObject* pl = get_attr(st, k_pages);
    if (!pl) {
      Py_DECREF(out);
      goto fail;
    }
    const Py_ssize_t np = PyObject_Length(pl);
    Py_DECREF(pl);
    if (np < 0) {
      Py_DECREF(out);
      goto fail;
    }
    const long after = seq + sl;
    long want = after > 0 ? (after + ps - 1) / ps : 0;
    long k = want - (long)np;
    if (k < 0) k = 0;
    need[i] = (int32_t)k;
    total += k;
  }
  Py_DECREF(sf);
  Py_XDECREF(lf);
  PyObject* res = Py_BuildValue("(LN)", total, out);
  return res;
fail:
  Py_DECREF(sf);
  Py_XDECREF(lf);
  return NULL;
}

/* Growable int32 buffer for the new-page tail of the metadata. */
typedef struct {
  int32_t* p;
  Py_ssize_t n, cap;
} ibuf;

static int ibuf_push(ibuf* b, long v) {
  if (b->n == b->cap) {
    Py_ssize_t cap = b->cap ? 2 * b->cap : 256;
    int32_t* q = (int32_t*)realloc(b->p, (size_t)cap * 4);
    if (!q) {
      PyErr_NoMemory();
      return -1;
    }
    b->p = q;
    b->cap = cap;
  }
  b->p[b->n++] = (int32_t)v;
  return 0;
}

/* Page id pl[j] of a list as a C long (-1 with an exception on error). */
static long page_at(PyObject* pl, Py_ssize_t j) {
  return PyLong_AsLong(PyList_GET_ITEM(pl, j));
}

/* (pl[0], pl[n-1]) as a new tuple, or (-1, -1) for an empty list. */
static PyObject* ends_of(PyObject* pl, Py_ssize_t n) {
  if (n == 0) return Py_BuildValue("(ii)", -1, -1);
  PyObject* a = PyList_GET_ITEM(pl, 0);
  PyObject* b = PyList_GET_ITEM(pl, n - 1);
  return PyTuple_Pack(2, a, b);
}

/* Whether (pl[0], pl[m-1]) equals the tuple `ends` (1), not (0), error (-1). */
static int ends_match(PyObject* pl, Py_ssize_t m, PyObject* ends) {
  if (!PyTuple_Check(ends) || PyTuple_GET_SIZE(ends) != 2) return 0;
  int r = PyObject_RichCompareBool(PyList_GET_ITEM(pl, 0), PyTuple_GET_ITEM(ends, 0), Py_EQ);
  if (r <= 0) return r;
  return PyObject_RichCompareBool(PyList_GET_ITEM(pl, m - 1), PyTuple_GET_ITEM(ends, 1), Py_EQ);
}

/* extend_meta(states, seq_lens, need, pages, stride, acquire) -> bytearray
 *
 * Hands pages (a list, or None when the caller already extended the lists)
 * out in request order: state i takes the next need[i] pages.  Then, per
 * state: acquire(state) when it has no block-table slot yet, the number of
 * leading pages the device row already holds (the DeviceBlockTable sync
 * rule: the synced list object, not shorter than then, with its first page
 * and its last synced page unchanged; otherwise 0), marking the state synced.
 * Returns the pack kernel's int32 metadata
 * [slot | seq_len | new_len | num_pages | pages on the device] (n each)
 * followed by every state's pages not yet on the device, in request order. */
static PyObject* py_extend_meta(PyObject* self, PyObject* args) {
  PyObject *states, *seq_lens, *need_obj, *pages, *acquire;
  long stride;
  if (!PyArg_ParseTuple(args, "OOOOlO", &states, &seq_lens, &need_obj, &pages, &stride, &acquire)) return NULL;
  PyObject* sf = PySequence_Fast(states, "states must be a sequence");
  if (!sf) return NULL;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(sf);
  PyObject* lf = NULL;
  PyObject* res = NULL;
  Py_buffer nb = {0};
  int have_nb = 0;
  ibuf tail = {0};
  int32_t* meta = NULL;
  if (seq_lens != Py_None) {
    lf = PySequence_Fast(seq_lens, "seq_lens must be a sequence");
    if (!lf) goto done;
    if (PySequence_Fast_GET_SIZE(lf) != n) {
      PyErr_Format(PyExc_ValueError, "%zd seq_lens for %zd states", PySequence_Fast_GET_SIZE(lf), n);
      goto done;
    }
  }
  if (pages != Py_None) {
    if (!PyList_Check(pages)) {
      PyErr_SetString(PyExc_TypeError, "pages must be a list");
      goto done;
    }
    if (PyObject_GetBuffer(need_obj, &nb, PyBUF_SIMPLE) < 0) goto done;
    have_nb = 1;
    if (nb.len != 4 * n) {
      PyErr_SetString(PyExc_ValueError, "need must hold one int32 per state");
      goto done;
    }
    const int32_t* need = (const int32_t*)nb.buf;
    Py_ssize_t off = 0;
    const Py_ssize_t avail = PyList_GET_SIZE(pages);
    for (Py_ssize_t i = 0; i < n; ++i) {
      const int32_t k = need[i];
      if (k <= 0) continue;
      if (off + k > avail) {
        PyErr_SetString(PyExc_ValueError, "fewer pages than the needs add up to");
        goto done;
      }
      PyObject* pl = get_attr(PySequence_Fast_GET_ITEM(sf, i), k_pages);
      if (!pl) goto done;
      PyObject* part = PyList_GetSlice(pages, off, off + k);
      int r = -1;
      if (part && PyList_Check(pl)) {
        r = PyList_SetSlice(pl, PY_SSIZE_T_MAX, PY_SSIZE_T_MAX, part);  /* pl.extend(part) */
      } else if (part) {
        PyObject* x = PyObject_CallMethod(pl, "extend", "O", part);
        r = x ? 0 : -1;
        Py_XDECREF(x);
      }
      Py_XDECREF(part);
      Py_DECREF(pl);
      if (r < 0) goto done;
      off += k;
    }
  }
  meta = (int32_t*)malloc((size_t)(5 * (n > 0 ? n : 1)) * 4);
  if (!meta) {
    PyErr_NoMemory();
    goto done;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* st = PySequence_Fast_GET_ITEM(sf, i);
    long slot, seq, sl;
    if (get_long(st, k_slot, &slot)) goto done;
    if (slot < 0) {
      PyObject* x = PyObject_CallFunctionObjArgs(acquire, st, NULL);
      if (!x) goto done;
      Py_DECREF(x);
      if (get_long(st, k_slot, &slot)) goto done;
    }
    if (get_long(st, k_seq_len, &seq) || seq_item(lf, i, &sl)) goto done;
    PyObject* pl = get_attr(st, k_pages);
    if (!pl) goto done;
    if (!PyList_Check(pl)) {
      Py_DECREF(pl);
      PyErr_SetString(PyExc_TypeError, "page_indices must be a list");
      goto done;
    }
    const Py_ssize_t np = PyList_GET_SIZE(pl);
    PyObject* dl = get_attr(st, k_dev_list);
    PyObject* de = NULL;
    long dlen = 0;
    Py_ssize_t start = 0;
    int synced = 0, bad = !dl || get_long(st, k_dev_len, &dlen) || !(de = get_attr(st, k_dev_ends));
    if (!bad && dl == pl && dlen <= np) {  /* the synced list object, not shorter than then */
      int ok = 1;
      if (dlen > 0) {  /* its first page and last synced page unchanged */
        ok = ends_match(pl, (Py_ssize_t)dlen, de);
        bad = ok < 0;
      }
      if (ok > 0) {
        start = (Py_ssize_t)dlen;
        synced = start == np;  /* nothing new (most requests of a decode step) */
      }
    }
    Py_XDECREF(dl);
    Py_XDECREF(de);
    if (bad) {
      Py_DECREF(pl);
      goto done;
    }
    if (!synced) {
      if (np > stride) {
        Py_DECREF(pl);
        PyErr_Format(PyExc_ValueError, "request holds %zd pages, block table rows hold %ld", np, stride);
        goto done;
      }
      for (Py_ssize_t j = start; j < np; ++j) {
        const long pg = page_at(pl, j);
        if ((pg == -1 && PyErr_Occurred()) || ibuf_push(&tail, pg)) {
          Py_DECREF(pl);
          goto done;
        }
      }
      PyObject* ends = ends_of(pl, np);
      int r = ends ? set_attr(st, k_dev_list, pl) : -1;
      if (!r) r = set_long(st, k_dev_len, (long)np);
      if (!r) r = set_attr(st, k_dev_ends, ends);
      Py_XDECREF(ends);
      if (r) {
        Py_DECREF(pl);
        goto done;
      }
    }
    Py_DECREF(pl);
    meta[i] = (int32_t)slot;
    meta[n + i] = (int32_t)seq;
    meta[2 * n + i] = (int32_t)sl;
    meta[3 * n + i] = (int32_t)np;
    meta[4 * n + i] = (int32_t)start;
  }
  res = PyByteArray_FromStringAndSize(NULL, (Py_ssize_t)(4 * (5 * n + tail.n)));
  if (res) {
    char* dst = PyByteArray_AS_STRING(res);
    memcpy(dst, meta, (size_t)(4 * 5 * n));
    if (tail.n) memcpy(dst + 4 * 5 * n, tail.p, (size_t)(4 * tail.n));
  }
done:
  if (have_nb) PyBuffer_Release(&nb);
  free(meta);
  free(tail.p);
  Py_DECREF(sf);
  Py_XDECREF(lf);
  return res;
}

/* advance(states, seq_lens, pos_advance): seq_len += seq_lens[i] and
 * position_id_start += pos_advance[i] (pos_advance None: seq_lens). */
static PyObject* py_advance(PyObject* self, PyObject* args) {
  PyObject *states, *seq_lens, *adv;
  if (!PyArg_ParseTuple(args, "OOO", &states, &seq_lens, &adv)) return NULL;
  PyObject* sf = PySequence_Fast(states, "states must be a sequence");
  if (!sf) return NULL;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(sf);
  PyObject* lf = PySequence_Fast(seq_lens, "seq_lens must be a sequence");
  PyObject* af = NULL;
  PyObject* res = NULL;
  if (!lf) goto done;
  if (adv != Py_None) {
    af = PySequence_Fast(adv, "pos_advance must be a sequence");
    if (!af) goto done;
  }
  /* zip() semantics of the Python loop: the shortest sequence bounds it */
  Py_ssize_t m = n < PySequence_Fast_GET_SIZE(lf) ? n : PySequence_Fast_GET_SIZE(lf);
  if (af && PySequence_Fast_GET_SIZE(af) < m) m = PySequence_Fast_GET_SIZE(af);
  for (Py_ssize_t i = 0; i < m; ++i) {
    PyObject* st = PySequence_Fast_GET_ITEM(sf, i);
    PyObject* d = PySequence_Fast_GET_ITEM(lf, i);
    PyObject* a = af ? PySequence_Fast_GET_ITEM(af, i) : d;
    PyObject* s0 = get_attr(st, k_seq_len);
    if (!s0) goto done;
    PyObject* s1 = PyNumber_Add(s0, d);
    Py_DECREF(s0);
    if (!s1 || set_attr(st, k_seq_len, s1)) {
      Py_XDECREF(s1);
      goto done;
    }
    Py_DECREF(s1);
    PyObject* p0 = get_attr(st, k_pos);
    if (!p0) goto done;
    PyObject* p1 = PyNumber_Add(p0, a);
    Py_DECREF(p0);
    if (!p1 || set_attr(st, k_pos, p1)) {
      Py_XDECREF(p1);
      goto done;
    }
    Py_DECREF(p1);
  }
  res = Py_None;
  Py_INCREF(res);
done:
  Py_DECREF(sf);
  Py_XDECREF(lf);
  Py_XDECREF(af);
  return res;
}

static PyMethodDef methods[] = {
    {"needs", py_needs, METH_VARARGS, "Per-state page need of one step: (total, int32 bytearray)."},
    {"extend_meta", py_extend_meta, METH_VARARGS, "Hand out pages, sync rule, pack metadata (int32 bytearray)."},
    {"advance", py_advance, METH_VARARGS, "seq_len and position_id_start advance over states."},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, MI_STR(MI_HOST_STEP_MODULE), NULL, -1, methods, NULL, NULL,
                                     NULL, NULL};

PyMODINIT_FUNC MI_CAT(PyInit_, MI_HOST_STEP_MODULE)(void) {
  k_seq_len = PyUnicode_InternFromString("seq_len");
  k_pos = PyUnicode_InternFromString("position_id_start");
  k_pages = PyUnicode_InternFromString("page_indices");
  k_slot = PyUnicode_InternFromString("slot");
  k_dev_list = PyUnicode_InternFromString("_dev_list");
  k_dev_len = PyUnicode_InternFromString("_dev_len");
  k_dev_ends = PyUnicode_InternFromString("_dev_ends");
  if (!k_seq_len || !k_pos || !k_pages || !k_slot || !k_dev_list || !k_dev_len || !k_dev_ends) return NULL;
  return PyModule_Create(&module);
}
