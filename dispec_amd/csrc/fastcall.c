/* CPython bindings of the C-ABI entry points that a decode step calls once per layer.
 *
 * ctypes converts each of a call's ~30 arguments through its argtypes before calling,
 * about 4-5 us per call, which is most of a small decode launch's host time.  These
 * METH_FASTCALL functions take the same positional arguments as the ctypes functions of
 * dispec_amd._lib (device pointers and sizes as Python ints, None for a null pointer, the
 * scale as a float) and call the library's entry points through the addresses that
 * dispec_amd._lib hands to bind(), so both paths reach the same loaded libdispec_hip.so.
 * Each returns the entry point's int status and, like ctypes, releases the GIL for the
 * duration of the call.  Built with gcc (no device code).
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stddef.h>
#include <stdint.h>

typedef union {
  void* p;
  int64_t q;
  int32_t i;
  float f;
  size_t z;
} arg_t;

/* Convert args[0..n) by the type letters of sig: P pointer (None -> NULL), q int64,
 * i int32, z size_t, f float.  Returns 0 with a Python error set on failure. */
static int convert(const char* name, const char* sig, PyObject* const* args, Py_ssize_t n,
                   arg_t* out) {
  const Py_ssize_t want = (Py_ssize_t)strlen(sig);
  if (n != want) {
    PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", name, want, n);
    return 0;
  }
  for (Py_ssize_t k = 0; k < n; ++k) {
    PyObject* o = args[k];
    switch (sig[k]) {
      case 'P':
        out[k].p = o == Py_None ? NULL : PyLong_AsVoidPtr(o);
        break;
      case 'q':
        out[k].q = PyLong_AsLongLong(o);
        break;
      case 'i':
        out[k].i = (int32_t)PyLong_AsLongLong(o);
        break;
      case 'z':
        out[k].z = (size_t)PyLong_AsUnsignedLongLong(o);
        break;
      case 'f':
        out[k].f = (float)PyFloat_AsDouble(o);
        break;
    }
    if (PyErr_Occurred()) {
      PyErr_Format(PyExc_TypeError, "%s: argument %zd has the wrong type", name, k);
      return 0;
    }
  }
  return 1;
}

/* ---- prototypes of include/dispec_hip.h (stream as void*) */
typedef int (*decode_fn)(void*, int64_t, int64_t, void*, void*, int64_t, int64_t, int64_t,
                         void*, int64_t, int32_t, void*, int64_t, void*, int32_t, int32_t,
                         int32_t, int32_t, float, int32_t, int32_t, void*, size_t, void*,
                         int64_t, int64_t, int32_t, void*, void*);
typedef int (*append_fn)(void*, void*, int64_t, int64_t, void*, void*, int64_t, void*, int64_t,
                         int64_t, void*, void*);
typedef int (*mq_fn)(void*, int64_t, int64_t, void*, void*, int64_t, int64_t, int64_t, void*,
                     int64_t, int32_t, void*, void*, int32_t, int32_t, int32_t, int32_t, float,
                     int32_t, int32_t, int32_t, void*, size_t, void*, int64_t, int64_t, int32_t,
                     void*, void*);
typedef int (*mq_sp_fn)(void*, int64_t, int64_t, void*, void*, int64_t, int64_t, int64_t, void*,
                        int64_t, int32_t, void*, void*, int32_t, int32_t, int32_t, int32_t,
                        float, int32_t, int32_t, int32_t, int32_t, void*, size_t, void*,
                        int64_t, int64_t, int32_t, void*, void*);
typedef int (*prologue_fn)(void*, int64_t, int64_t, void*, int64_t, int64_t, void*, int64_t,
                           int64_t, void*, void*, float, void*, void*, int64_t, void*, int64_t,
                           int32_t, int32_t, int32_t, void*, int64_t, int64_t, void*, void*,
                           int64_t, int64_t, int64_t, int32_t, void*, void*);

static decode_fn p_decode;
static append_fn p_append;
static mq_fn p_mq;
static mq_sp_fn p_mq_sp;
static prologue_fn p_prologue;

#define UNBOUND(ptr, name)                                                        \
  if (!(ptr)) {                                                                   \
    PyErr_SetString(PyExc_RuntimeError, name " is not bound (call bind first)"); \
    return NULL;                                                                  \
  }

static const char kDecodeSig[] = "PqqPPqqqPqiPqPiiiifiiPzPqqiPP";
static PyObject* w_decode(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  arg_t v[32];
  UNBOUND(p_decode, "dsp_paged_decode");
  if (!convert("dsp_paged_decode", kDecodeSig, a, n, v)) return NULL;
  int st;
  Py_BEGIN_ALLOW_THREADS
  st = p_decode(v[0].p, v[1].q, v[2].q, v[3].p, v[4].p, v[5].q, v[6].q,
                v[7].q, v[8].p, v[9].q, v[10].i, v[11].p, v[12].q, v[13].p,
                v[14].i, v[15].i, v[16].i, v[17].i, v[18].f, v[19].i, v[20].i,
                v[21].p, v[22].z, v[23].p, v[24].q, v[25].q, v[26].i, v[27].p,
                v[28].p);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(st);
}

static const char kAppendSig[] = "PPqqPPqPqqPP";
static PyObject* w_append(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  arg_t v[16];
  UNBOUND(p_append, "dsp_kv_append");
  if (!convert("dsp_kv_append", kAppendSig, a, n, v)) return NULL;
  int st;
  Py_BEGIN_ALLOW_THREADS
  st = p_append(v[0].p, v[1].p, v[2].q, v[3].q, v[4].p, v[5].p, v[6].q,
                v[7].p, v[8].q, v[9].q, v[10].p, v[11].p);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(st);
}

static const char kMqSig[] = "PqqPPqqqPqiPPiiiifiiiPzPqqiPP";
static PyObject* w_mq(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  arg_t v[32];
  UNBOUND(p_mq, "dsp_paged_mq_attention");
  if (!convert("dsp_paged_mq_attention", kMqSig, a, n, v)) return NULL;
  int st;
  Py_BEGIN_ALLOW_THREADS
  st = p_mq(v[0].p, v[1].q, v[2].q, v[3].p, v[4].p, v[5].q, v[6].q, v[7].q,
            v[8].p, v[9].q, v[10].i, v[11].p, v[12].p, v[13].i, v[14].i,
            v[15].i, v[16].i, v[17].f, v[18].i, v[19].i, v[20].i, v[21].p,
            v[22].z, v[23].p, v[24].q, v[25].q, v[26].i, v[27].p, v[28].p);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(st);
}

static const char kMqSpSig[] = "PqqPPqqqPqiPPiiiifiiiiPzPqqiPP";
static PyObject* w_mq_sp(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  arg_t v[32];
  UNBOUND(p_mq_sp, "dsp_paged_mq_attention_shared_prefix");
  if (!convert("dsp_paged_mq_attention_shared_prefix", kMqSpSig, a, n, v)) return NULL;
  int st;
  Py_BEGIN_ALLOW_THREADS
  st = p_mq_sp(v[0].p, v[1].q, v[2].q, v[3].p, v[4].p, v[5].q, v[6].q,
               v[7].q, v[8].p, v[9].q, v[10].i, v[11].p, v[12].p, v[13].i,
               v[14].i, v[15].i, v[16].i, v[17].f, v[18].i, v[19].i, v[20].i,
               v[21].i, v[22].p, v[23].z, v[24].p, v[25].q, v[26].q, v[27].i,
               v[28].p, v[29].p);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(st);
}

static const char kPrologueSig[] = "PqqPqqPqqPPfPPqPqiiiPqqPPqqqiPP";
static PyObject* w_prologue(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  arg_t v[32];
  UNBOUND(p_prologue, "dsp_qk_norm_rope_append");
  if (!convert("dsp_qk_norm_rope_append", kPrologueSig, a, n, v)) return NULL;
  int st;
  Py_BEGIN_ALLOW_THREADS
  st = p_prologue(v[0].p, v[1].q, v[2].q, v[3].p, v[4].q, v[5].q, v[6].p,
                  v[7].q, v[8].q, v[9].p, v[10].p, v[11].f, v[12].p, v[13].p,
                  v[14].q, v[15].p, v[16].q, v[17].i, v[18].i, v[19].i,
                  v[20].p, v[21].q, v[22].q, v[23].p, v[24].p, v[25].q, v[26].q,
                  v[27].q, v[28].i, v[29].p, v[30].p);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(st);
}

/* bind(name, address): the entry point `name` of the loaded library is at `address`. */
static PyObject* w_bind(PyObject* self, PyObject* args) {
  const char* name;
  unsigned long long addr;
  if (!PyArg_ParseTuple(args, "sK", &name, &addr)) return NULL;
  void* p = (void*)(uintptr_t)addr;
  if (!strcmp(name, "dsp_paged_decode")) p_decode = (decode_fn)p;
  else if (!strcmp(name, "dsp_kv_append")) p_append = (append_fn)p;
  else if (!strcmp(name, "dsp_paged_mq_attention")) p_mq = (mq_fn)p;
  else if (!strcmp(name, "dsp_paged_mq_attention_shared_prefix")) p_mq_sp = (mq_sp_fn)p;
  else if (!strcmp(name, "dsp_qk_norm_rope_append")) p_prologue = (prologue_fn)p;
  else {
    PyErr_Format(PyExc_KeyError, "no fast binding for %s", name);
    return NULL;
  }
  Py_RETURN_NONE;
}

static PyMethodDef kMethods[] = {
    {"bind", w_bind, METH_VARARGS, "bind(name, address) -> None"},
    {"dsp_paged_decode", (PyCFunction)(void (*)(void))w_decode, METH_FASTCALL, NULL},
    {"dsp_kv_append", (PyCFunction)(void (*)(void))w_append, METH_FASTCALL, NULL},
    {"dsp_paged_mq_attention", (PyCFunction)(void (*)(void))w_mq, METH_FASTCALL, NULL},
    {"dsp_paged_mq_attention_shared_prefix", (PyCFunction)(void (*)(void))w_mq_sp,
     METH_FASTCALL, NULL},
    {"dsp_qk_norm_rope_append", (PyCFunction)(void (*)(void))w_prologue, METH_FASTCALL, NULL},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_fastcall", NULL, -1, kMethods};

/* The module exports SIGNATURES = {name: type letters}, the argument types each function
 * converts, so the loader can compare them with its ctypes argtypes and refuse to bind a
 * function whose prototype here has fallen out of step with the header. */
PyMODINIT_FUNC PyInit__fastcall(void) {
  static const struct {
    const char* name;
    const char* sig;
  } kSigs[] = {{"dsp_paged_decode", kDecodeSig},
               {"dsp_kv_append", kAppendSig},
               {"dsp_paged_mq_attention", kMqSig},
               {"dsp_paged_mq_attention_shared_prefix", kMqSpSig},
               {"dsp_qk_norm_rope_append", kPrologueSig}};
  PyObject* m = PyModule_Create(&kModule);
  if (!m) return NULL;
  PyObject* sigs = PyDict_New();
  if (!sigs) goto fail;
  for (size_t k = 0; k < sizeof(kSigs) / sizeof(kSigs[0]); ++k) {
    PyObject* v = PyUnicode_FromString(kSigs[k].sig);
    if (!v || PyDict_SetItemString(sigs, kSigs[k].name, v) < 0) {
      Py_XDECREF(v);
      Py_DECREF(sigs);
      goto fail;
    }
    Py_DECREF(v);
  }
  if (PyModule_AddObject(m, "SIGNATURES", sigs) < 0) {
    Py_DECREF(sigs);
    goto fail;
  }
  return m;
fail:
  Py_DECREF(m);
  return NULL;
}
