/*
 * _glue: CPython calls into libactkv_hip.so's hot entry points without ctypes.
 *
 * A ctypes call converts every argument through its argtype object (about
 * 0.1 us per argument); the scoring, keep-mask and compaction entry points take
 * 26-38 arguments each, so an eviction step spent several microseconds of host
 * time on argument conversion alone.  Here each entry point has a METH_FASTCALL
 * wrapper that converts its arguments with the C API and calls the library
 * through a function pointer of the exact prototype in include/actkv.h.
 *
 * The module does not link the library: actkv/_hip.py loads the library with
 * ctypes (one copy per process) and hands the entry points' addresses to
 * bind().  Argument rules match ctypes: pointers are ints or None (NULL),
 * integers must fit their C type (OverflowError otherwise), floats are
 * converted to float.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <string.h>

#include "actkv.h"

/* hipMemcpyAsync(dst, src, bytes, kind, stream): the HIP runtime the library links */
typedef int (*memcpy_async_fn)(void *, const void *, size_t, int, void *);

static __typeof__(&actkv_action_scores) p_action_scores;
static __typeof__(&actkv_keep_mask) p_keep_mask;
static __typeof__(&actkv_compact) p_compact;
static memcpy_async_fn p_memcpy_async;

typedef union {
  void *p;
  int64_t l;
  int32_t i;
  size_t z;
  float f;
} Arg;

/* Re-raise the pending conversion error with the entry point and argument named. */
static int arg_error(const char *name, Py_ssize_t k) {
  PyObject *type, *value, *tb;
  PyErr_Fetch(&type, &value, &tb);
  PyErr_Format(type ? type : PyExc_TypeError, "%s: argument %zd: %S", name, k, value ? value : Py_None);
  Py_XDECREF(type);
  Py_XDECREF(value);
  Py_XDECREF(tb);
  return -1;
}

/* Signature letters: p pointer (int or None), l int64, i int32, z size_t, f float. */
static int convert(const char *name, const char *sig, PyObject *const *args, Py_ssize_t n,
                   Arg *out) {
  const Py_ssize_t want = (Py_ssize_t)strlen(sig);
  if (n != want) {
    PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", name, want, n);
    return -1;
  }
  for (Py_ssize_t k = 0; k < n; ++k) {
    PyObject *o = args[k];
    switch (sig[k]) {
      case 'p':
        if (o == Py_None) {
          out[k].p = NULL;
        } else {
          out[k].p = PyLong_AsVoidPtr(o);
          if (out[k].p == NULL && PyErr_Occurred()) return arg_error(name, k);
        }
        break;
      case 'l':
        out[k].l = PyLong_AsLongLong(o);
        if (out[k].l == -1 && PyErr_Occurred()) return arg_error(name, k);
        break;
      case 'i': {
        const long long v = PyLong_AsLongLong(o);
        if (v == -1 && PyErr_Occurred()) return arg_error(name, k);
        if (v < INT32_MIN || v > INT32_MAX) {
          PyErr_Format(PyExc_OverflowError, "%s: argument %zd (%lld) does not fit a C int", name, k, v);
          return -1;
        }
        out[k].i = (int32_t)v;
        break;
      }
      case 'z':
        out[k].z = PyLong_AsSize_t(o);
        if (out[k].z == (size_t)-1 && PyErr_Occurred()) return arg_error(name, k);
        break;
      case 'f': {
        const double d = PyFloat_AsDouble(o);
        if (d == -1.0 && PyErr_Occurred()) return arg_error(name, k);
        out[k].f = (float)d;
        break;
      }
      default:
        PyErr_Format(PyExc_SystemError, "%s: bad signature letter", name);
        return -1;
    }
  }
  return 0;
}

static int unbound(const void *fn, const char *name) {
  if (fn) return 0;
  PyErr_Format(PyExc_RuntimeError, "_glue.%s called before bind()", name);
  return -1;
}

#define SIG_ACTION_SCORES "pillll" "pillll" "l" "pli" "p" "plll" "pllll" "ppp" "iiiiiii" "fp"
#define SIG_KEEP_MASK "pilll" "iii" "ppppl" "i" "plpl" "iipzp"
#define SIG_COMPACT "plllll" "plip" "pli" "plplppl" "plpl" "pplp" "iiip"
#define SIG_MEMCPY "ppzip"

static PyObject *g_action_scores(PyObject *self, PyObject *const *args, Py_ssize_t n) {
  Arg a[38];
  if (unbound((const void *)p_action_scores, "action_scores") ||
      convert("actkv_action_scores", SIG_ACTION_SCORES, args, n, a))
    return NULL;
  const int rc = p_action_scores(
      a[0].p, a[1].i, a[2].l, a[3].l, a[4].l, a[5].l,
      a[6].p, a[7].i, a[8].l, a[9].l, a[10].l, a[11].l,
      a[12].l,
      (const int32_t *)a[13].p, a[14].l, a[15].i,
      (const int32_t *)a[16].p,
      (const float *)a[17].p, a[18].l, a[19].l, a[20].l,
      (float *)a[21].p, a[22].l, a[23].l, a[24].l, a[25].l,
      (int32_t *)a[26].p, (const int32_t *)a[27].p, (const int32_t *)a[28].p,
      a[29].i, a[30].i, a[31].i, a[32].i, a[33].i, a[34].i, a[35].i,
      a[36].f, a[37].p);
  return PyLong_FromLong(rc);
}

static PyObject *g_keep_mask(PyObject *self, PyObject *const *args, Py_ssize_t n) {
  Arg a[26];
  if (unbound((const void *)p_keep_mask, "keep_mask") ||
      convert("actkv_keep_mask", SIG_KEEP_MASK, args, n, a))
    return NULL;
  const int rc = p_keep_mask(
      a[0].p, a[1].i, a[2].l, a[3].l, a[4].l,
      a[5].i, a[6].i, a[7].i,
      (const int32_t *)a[8].p, (const int32_t *)a[9].p, (const int32_t *)a[10].p,
      (const uint8_t *)a[11].p, a[12].l,
      a[13].i,
      (uint8_t *)a[14].p, a[15].l, (uint32_t *)a[16].p, a[17].l,
      a[18].i, a[19].i, a[20].p, a[21].z, a[22].p);
  return PyLong_FromLong(rc);
}

static PyObject *g_compact(PyObject *self, PyObject *const *args, Py_ssize_t n) {
  Arg a[33];
  if (unbound((const void *)p_compact, "compact") || convert("actkv_compact", SIG_COMPACT, args, n, a))
    return NULL;
  const int rc = p_compact(
      a[0].p, a[1].l, a[2].l, a[3].l, a[4].l, a[5].l,
      (const uint32_t *)a[6].p, a[7].l, a[8].i, (const int32_t *)a[9].p,
      (const int32_t *)a[10].p, a[11].l, a[12].i,
      (int64_t *)a[13].p, a[14].l, (const uint8_t *)a[15].p, a[16].l,
      (const int32_t *)a[17].p, (uint8_t *)a[18].p, a[19].l,
      (int32_t *)a[20].p, a[21].l, (int32_t *)a[22].p, a[23].l,
      (int64_t *)a[24].p, (int64_t *)a[25].p, a[26].l, (int32_t *)a[27].p,
      a[28].i, a[29].i, a[30].i, a[31].p);
  return PyLong_FromLong(rc);
}

static PyObject *g_memcpy_async(PyObject *self, PyObject *const *args, Py_ssize_t n) {
  Arg a[5];
  if (unbound((const void *)p_memcpy_async, "memcpy_async") ||
      convert("hipMemcpyAsync", SIG_MEMCPY, args, n, a))
    return NULL;
  return PyLong_FromLong(p_memcpy_async(a[0].p, a[1].p, a[2].z, a[3].i, a[4].p));
}

/* bind(action_scores, keep_mask, compact, memcpy_async): the entry points' addresses */
static PyObject *g_bind(PyObject *self, PyObject *const *args, Py_ssize_t n) {
  Arg a[4];
  if (convert("bind", "pppp", args, n, a)) return NULL;
  for (int k = 0; k < 4; ++k)
    if (!a[k].p) {
      PyErr_SetString(PyExc_ValueError, "bind: NULL entry point");
      return NULL;
    }
  p_action_scores = (__typeof__(p_action_scores))a[0].p;
  p_keep_mask = (__typeof__(p_keep_mask))a[1].p;
  p_compact = (__typeof__(p_compact))a[2].p;
  p_memcpy_async = (memcpy_async_fn)a[3].p;
  Py_RETURN_NONE;
}

/* signatures(): {entry point: letters}, for checking against the ctypes declarations */
static PyObject *g_signatures(PyObject *self, PyObject *unused) {
  return Py_BuildValue("{ssssssss}", "actkv_action_scores", SIG_ACTION_SCORES, "actkv_keep_mask",
                       SIG_KEEP_MASK, "actkv_compact", SIG_COMPACT, "hipMemcpyAsync", SIG_MEMCPY);
}

static PyMethodDef methods[] = {
    {"bind", (PyCFunction)(void (*)(void))g_bind, METH_FASTCALL, "bind the library's entry points"},
    {"action_scores", (PyCFunction)(void (*)(void))g_action_scores, METH_FASTCALL, "actkv_action_scores"},
    {"keep_mask", (PyCFunction)(void (*)(void))g_keep_mask, METH_FASTCALL, "actkv_keep_mask"},
    {"compact", (PyCFunction)(void (*)(void))g_compact, METH_FASTCALL, "actkv_compact"},
    {"memcpy_async", (PyCFunction)(void (*)(void))g_memcpy_async, METH_FASTCALL, "hipMemcpyAsync"},
    {"signatures", g_signatures, METH_NOARGS, "argument letters of each wrapped entry point"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_glue",
                                    "CPython calls into libactkv_hip.so's hot entry points", -1, methods,
                                    NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__glue(void) { return PyModule_Create(&module); }
