/*
 * fdcall.c - CPython binding of the C ABI in include/fused_decode.h.
 *
 * The operators launch one or two small kernels per call, and at one token the
 * host side of a call (argument conversion, the HIP launch) is as long as the
 * kernel itself. ctypes spends about 0.15 us per argument converting Python
 * ints; this module takes the same arguments through METH_FASTCALL and calls
 * the library directly, for a few tens of nanoseconds per argument. It knows
 * nothing of torch: pointers arrive as Python ints (tensor.data_ptr()), the
 * fd_rows / fd_tile structs as bytes objects of their exact size, the stream
 * as an int (hipStream_t).
 *
 * bind(path) dlopens libfused_decode_hip.so (the same file ctypes loads, so
 * both share one copy of the library and its per-thread error string) and
 * resolves every entry point; the wrappers return the int status unchanged.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <dlfcn.h>
#include <stdint.h>

#include "fused_decode.h"

typedef union {
  void* p;
  int64_t l;
  int i;
  float f;
} Arg;

/* Argument codes: p pointer (int or None), s stream (same), i int, l int64,
 * f float, r const fd_rows* (bytes of sizeof(fd_rows)), t const fd_tile*
 * (bytes of sizeof(fd_tile), or None). */
static int parse(const char* fn, PyObject* const* args, Py_ssize_t nargs, const char* fmt,
                 Arg* out) {
  const Py_ssize_t want = (Py_ssize_t)strlen(fmt);
  if (nargs != want) {
    PyErr_Format(PyExc_TypeError, "%s takes %zd arguments, got %zd", fn, want, nargs);
    return -1;
  }
  for (Py_ssize_t k = 0; k < want; ++k) {
    PyObject* o = args[k];
    switch (fmt[k]) {
      case 'p':
      case 's':
        out[k].p = o == Py_None ? NULL : PyLong_AsVoidPtr(o);
        break;
      case 'i':
        out[k].i = (int)PyLong_AsLong(o);
        break;
      case 'l':
        out[k].l = (int64_t)PyLong_AsLongLong(o);
        break;
      case 'f':
        out[k].f = (float)PyFloat_AsDouble(o);
        break;
      case 'r':
      case 't': {
        const Py_ssize_t size = fmt[k] == 'r' ? (Py_ssize_t)sizeof(fd_rows) : (Py_ssize_t)sizeof(fd_tile);
        if (fmt[k] == 't' && o == Py_None) {
          out[k].p = NULL;
          break;
        }
        if (!PyBytes_Check(o) || PyBytes_GET_SIZE(o) != size) {
          PyErr_Format(PyExc_TypeError, "%s argument %zd must be bytes of length %zd", fn, k, size);
          return -1;
        }
        out[k].p = PyBytes_AS_STRING(o);
        break;
      }
      default:
        PyErr_SetString(PyExc_SystemError, "bad argument code");
        return -1;
    }
    if (PyErr_Occurred()) return -1;
  }
  return 0;
}

/* Entry points, resolved by bind(). */
static void* g_handle;
static const char* (*p_last_error)(void);
static int (*p_version)(void);
static int (*p_rms_norm)(void*, const void*, const void*, int, int64_t, const fd_rows*,
                         const fd_rows*, float, int, void*);
static int (*p_add_rms_norm)(void*, void*, const void*, const void*, const void*, int, int64_t,
                             const fd_rows*, const fd_rows*, const fd_rows*, const fd_rows*, float,
                             int, void*);
static int (*p_swiglu)(void*, const void*, const void*, const fd_rows*, const fd_rows*,
                       const fd_rows*, int, void*);
static int (*p_rope)(void*, const void*, const void*, const void*, int, const fd_rows*,
                     const fd_rows*, const fd_rows*, const fd_rows*, int, void*);
static int (*p_linear_tiled)(void*, const void*, const void*, const void*, int, const void*, int,
                             int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                             int64_t, int64_t, int64_t, int64_t, int64_t, const fd_tile*, int, int,
                             void*);
static int (*p_post_attn_mlp)(void*, void*, const void*, const void*, int, const void*,
                              const void*, int64_t, int64_t, int64_t, float, int, int, void*);
static int (*p_pre_attn_qkv)(void*, void*, const void*, const void*, int, const void*, const void*,
                             int, const void*, const void*, int, int64_t, int64_t, int64_t,
                             int64_t, int64_t, int64_t, float, int, int, void*);
static int (*p_linear_fp8)(void*, const void*, const void*, const float*, const void*, int,
                           const void*, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                           int64_t, int64_t, int64_t, int64_t, int, void*);
static int (*p_post_attn_mlp_fp8)(void*, void*, const void*, const void*, int, const void*,
                                  const float*, const void*, const float*, int64_t, int64_t,
                                  int64_t, float, int, void*);
static int (*p_pre_attn_qkv_fp8)(void*, void*, const void*, const void*, int, const void*,
                                 const float*, const void*, int, const void*, const void*, int,
                                 int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, float, int,
                                 void*);
static int (*p_copy)(void*, const void*, int64_t, void*);
static int (*p_triad)(void*, const void*, const void*, float, int64_t, int, void*);
static int (*p_read)(const void*, int64_t, int, void*, void*);

#define NEED_BOUND()                                                           \
  if (!g_handle) {                                                             \
    PyErr_SetString(PyExc_RuntimeError, "fused_decode._fdcall: bind() first"); \
    return NULL;                                                               \
  }

#define WRAP(name, fmt, call)                                                         \
  static PyObject* w_##name(PyObject* self, PyObject* const* args, Py_ssize_t nargs) { \
    (void)self;                                                                       \
    Arg a[32];                                                                        \
    NEED_BOUND();                                                                     \
    if (parse(#name, args, nargs, fmt, a) < 0) return NULL;                           \
    return PyLong_FromLong((long)(call));                                             \
  }

WRAP(rms_norm, "pppilrrfis",
     p_rms_norm(a[0].p, a[1].p, a[2].p, a[3].i, a[4].l, (const fd_rows*)a[5].p,
                (const fd_rows*)a[6].p, a[7].f, a[8].i, a[9].p))
WRAP(add_rms_norm, "pppppilrrrrfis",
     p_add_rms_norm(a[0].p, a[1].p, a[2].p, a[3].p, a[4].p, a[5].i, a[6].l, (const fd_rows*)a[7].p,
                    (const fd_rows*)a[8].p, (const fd_rows*)a[9].p, (const fd_rows*)a[10].p,
                    a[11].f, a[12].i, a[13].p))
WRAP(swiglu, "ppprrris",
     p_swiglu(a[0].p, a[1].p, a[2].p, (const fd_rows*)a[3].p, (const fd_rows*)a[4].p,
              (const fd_rows*)a[5].p, a[6].i, a[7].p))
WRAP(rope, "ppppirrrris",
     p_rope(a[0].p, a[1].p, a[2].p, a[3].p, a[4].i, (const fd_rows*)a[5].p, (const fd_rows*)a[6].p,
            (const fd_rows*)a[7].p, (const fd_rows*)a[8].p, a[9].i, a[10].p))
WRAP(linear_tiled, "ppppipilllllllllllltiis",
     p_linear_tiled(a[0].p, a[1].p, a[2].p, a[3].p, a[4].i, a[5].p, a[6].i, a[7].l, a[8].l,
                    a[9].l, a[10].l, a[11].l, a[12].l, a[13].l, a[14].l, a[15].l, a[16].l, a[17].l,
                    a[18].l, (const fd_tile*)a[19].p, a[20].i, a[21].i, a[22].p))
WRAP(post_attn_mlp, "ppppipplllfiis",
     p_post_attn_mlp(a[0].p, a[1].p, a[2].p, a[3].p, a[4].i, a[5].p, a[6].p, a[7].l, a[8].l,
                     a[9].l, a[10].f, a[11].i, a[12].i, a[13].p))
WRAP(pre_attn_qkv, "ppppippippillllllfiis",
     p_pre_attn_qkv(a[0].p, a[1].p, a[2].p, a[3].p, a[4].i, a[5].p, a[6].p, a[7].i, a[8].p,
                    a[9].p, a[10].i, a[11].l, a[12].l, a[13].l, a[14].l, a[15].l, a[16].l,
                    a[17].f, a[18].i, a[19].i, a[20].p))
WRAP(linear_fp8, "pppppipillllllllllis",
     p_linear_fp8(a[0].p, a[1].p, a[2].p, (const float*)a[3].p, a[4].p, a[5].i, a[6].p, a[7].i,
                  a[8].l, a[9].l, a[10].l, a[11].l, a[12].l, a[13].l, a[14].l, a[15].l, a[16].l,
                  a[17].l, a[18].i, a[19].p))
WRAP(post_attn_mlp_fp8, "ppppipppplllfis",
     p_post_attn_mlp_fp8(a[0].p, a[1].p, a[2].p, a[3].p, a[4].i, a[5].p, (const float*)a[6].p,
                         a[7].p, (const float*)a[8].p, a[9].l, a[10].l, a[11].l, a[12].f, a[13].i,
                         a[14].p))
WRAP(pre_attn_qkv_fp8, "ppppipppippillllllfis",
     p_pre_attn_qkv_fp8(a[0].p, a[1].p, a[2].p, a[3].p, a[4].i, a[5].p, (const float*)a[6].p,
                        a[7].p, a[8].i, a[9].p, a[10].p, a[11].i, a[12].l, a[13].l, a[14].l,
                        a[15].l, a[16].l, a[17].l, a[18].f, a[19].i, a[20].p))
WRAP(copy, "ppls", p_copy(a[0].p, a[1].p, a[2].l, a[3].p))
WRAP(triad, "pppflis", p_triad(a[0].p, a[1].p, a[2].p, a[3].f, a[4].l, a[5].i, a[6].p))
WRAP(read, "plips", p_read(a[0].p, a[1].l, a[2].i, a[3].p, a[4].p))

static PyObject* w_last_error(PyObject* self, PyObject* unused) {
  (void)self;
  (void)unused;
  NEED_BOUND();
  return PyUnicode_DecodeUTF8(p_last_error(), (Py_ssize_t)strlen(p_last_error()), "replace");
}

static PyObject* w_version(PyObject* self, PyObject* unused) {
  (void)self;
  (void)unused;
  NEED_BOUND();
  return PyLong_FromLong(p_version());
}

#define RESOLVE(var, sym)                                                                   \
  do {                                                                                      \
    *(void**)(&var) = dlsym(h, sym);                                                        \
    if (!var) {                                                                             \
      PyErr_Format(PyExc_ImportError, "%s does not export %s", path, sym);                  \
      dlclose(h);                                                                           \
      return NULL;                                                                          \
    }                                                                                       \
  } while (0)

static PyObject* w_bind(PyObject* self, PyObject* arg) {
  (void)self;
  const char* path = PyUnicode_AsUTF8(arg);
  if (!path) return NULL;
  if (g_handle) Py_RETURN_NONE;
  void* h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
  if (!h) {
    PyErr_Format(PyExc_ImportError, "cannot load %s: %s", path, dlerror());
    return NULL;
  }
  RESOLVE(p_last_error, "fd_last_error");
  RESOLVE(p_version, "fd_version");
  RESOLVE(p_rms_norm, "fd_rms_norm");
  RESOLVE(p_add_rms_norm, "fd_add_rms_norm");
  RESOLVE(p_swiglu, "fd_swiglu");
  RESOLVE(p_rope, "fd_rope");
  RESOLVE(p_linear_tiled, "fd_linear_tiled");
  RESOLVE(p_post_attn_mlp, "fd_post_attn_mlp");
  RESOLVE(p_pre_attn_qkv, "fd_pre_attn_qkv");
  RESOLVE(p_linear_fp8, "fd_linear_fp8");
  RESOLVE(p_post_attn_mlp_fp8, "fd_post_attn_mlp_fp8");
  RESOLVE(p_pre_attn_qkv_fp8, "fd_pre_attn_qkv_fp8");
  RESOLVE(p_copy, "fd_copy");
  RESOLVE(p_triad, "fd_triad");
  RESOLVE(p_read, "fd_read");
  g_handle = h;
  Py_RETURN_NONE;
}

#define FAST(name) {#name, (PyCFunction)(void (*)(void))w_##name, METH_FASTCALL, NULL}

static PyMethodDef methods[] = {
    {"bind", w_bind, METH_O, "bind(path): load the HIP library and resolve its entry points"},
    {"last_error", w_last_error, METH_NOARGS, "fd_last_error() of this thread"},
    {"version", w_version, METH_NOARGS, "fd_version()"},
    FAST(rms_norm),
    FAST(add_rms_norm),
    FAST(swiglu),
    FAST(rope),
    FAST(linear_tiled),
    FAST(post_attn_mlp),
    FAST(pre_attn_qkv),
    FAST(linear_fp8),
    FAST(post_attn_mlp_fp8),
    FAST(pre_attn_qkv_fp8),
    FAST(copy),
    FAST(triad),
    FAST(read),
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {
    PyModuleDef_HEAD_INIT, "_fdcall",
    "CPython binding of the fused_decode C ABI (see include/fused_decode.h).", -1, methods,
    NULL, NULL, NULL, NULL,
};

PyMODINIT_FUNC PyInit__fdcall(void) { return PyModule_Create(&module); }
