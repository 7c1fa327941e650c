/* _g16fast: a CPython extension that calls the per-call entry points of libg16.so that sit on
 * latency-bound paths -- g16_skinny_f32in and g16_skinny_strips_f32in (the FastLinear decode
 * shortcut, the counterpart of the reference's PreparedLaunch, src/gtx16_fp16/kernels.py:324-338)
 * and g16_mm_t_gemm (mm_t's GEMM path, ops.py:86-108) -- with METH_FASTCALL argument parsing. Through ctypes the same calls spend
 * ~0.1 us per argument converting them; here the conversion is a few ns per argument.
 *
 * The module does not link libg16.so: bind() receives the addresses of the three functions from the
 * library the ctypes binding already loaded, so both bindings call into the same instance. Pointer
 * arguments are Python ints or None (NULL); every call returns the entry point's int status. The
 * GIL is released around the call, as ctypes does.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stddef.h>
#include <stdint.h>

typedef int (*skinny_fn)(const void*, const void*, void*, const void*, int, int, int, int, void*, size_t, void*,
                         size_t, void*);
typedef int (*mm_t_gemm_fn)(const void*, int, const void*, void*, int, const void*, float, int, int, int, int, void*,
                            size_t, void*, size_t, void*, size_t, void*);

typedef int (*strips_fn)(const void*, const void*, void*, const void*, int, int, int, void*);
static skinny_fn g_skinny_f32in = NULL;
static strips_fn g_strips_f32in = NULL;
static mm_t_gemm_fn g_mm_t_gemm = NULL;

static int as_ptr(PyObject* o, void** out) {
  if (o == Py_None) {
    *out = NULL;
    return 0;
  }
  *out = PyLong_AsVoidPtr(o);
  return (*out == NULL && PyErr_Occurred()) ? -1 : 0;
}

static int as_int(PyObject* o, int* out) {
  const long v = PyLong_AsLong(o);
  if (v == -1 && PyErr_Occurred()) return -1;
  if (v < INT32_MIN || v > INT32_MAX) {
    PyErr_SetString(PyExc_OverflowError, "argument does not fit a C int");
    return -1;
  }
  *out = (int)v;
  return 0;
}

static int as_size(PyObject* o, size_t* out) {
  *out = PyLong_AsSize_t(o);
  return (*out == (size_t)-1 && PyErr_Occurred()) ? -1 : 0;
}

static int check_nargs(const char* name, Py_ssize_t nargs, Py_ssize_t want) {
  if (nargs == want) return 0;
  PyErr_Format(PyExc_TypeError, "%s() takes %zd arguments (%zd given)", name, want, nargs);
  return -1;
}

static PyObject* fast_bind(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  void *skinny, *gemm, *strips;
  if (check_nargs("bind", nargs, 3) || as_ptr(args[0], &skinny) || as_ptr(args[1], &gemm) ||
      as_ptr(args[2], &strips))
    return NULL;
  if (skinny == NULL || gemm == NULL || strips == NULL) {
    PyErr_SetString(PyExc_ValueError, "bind() needs three non-NULL function addresses");
    return NULL;
  }
  g_skinny_f32in = (skinny_fn)skinny;
  g_mm_t_gemm = (mm_t_gemm_fn)gemm;
  g_strips_f32in = (strips_fn)strips;
  Py_RETURN_NONE;
}

static int check_bound(const void* fn) {
  if (fn != NULL) return 0;
  PyErr_SetString(PyExc_RuntimeError, "_g16fast: bind() has not been called");
  return -1;
}

/* skinny_f32in(x, w_t, out, bias, M, N, K, ksplit, partials, partial_bytes, counters, counter_bytes,
 * stream) -> status of g16_skinny_f32in */
static PyObject* fast_skinny_f32in(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  void *x, *w, *out, *bias, *part, *cnt, *stream;
  int M, N, K, ksplit, st;
  size_t part_bytes, cnt_bytes;
  if (check_bound((const void*)g_skinny_f32in) || check_nargs("skinny_f32in", nargs, 13)) return NULL;
  if (as_ptr(args[0], &x) || as_ptr(args[1], &w) || as_ptr(args[2], &out) || as_ptr(args[3], &bias) ||
      as_int(args[4], &M) || as_int(args[5], &N) || as_int(args[6], &K) || as_int(args[7], &ksplit) ||
      as_ptr(args[8], &part) || as_size(args[9], &part_bytes) || as_ptr(args[10], &cnt) ||
      as_size(args[11], &cnt_bytes) || as_ptr(args[12], &stream))
    return NULL;
  Py_BEGIN_ALLOW_THREADS
  st = g_skinny_f32in(x, w, out, bias, M, N, K, ksplit, part, part_bytes, cnt, cnt_bytes, stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(st);
}

/* skinny_strips_f32in(x, wd, out, bias, M, N, K, stream) -> status of g16_skinny_strips_f32in */
static PyObject* fast_strips_f32in(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  void *x, *wd, *out, *bias, *stream;
  int M, N, K, st;
  if (check_bound((const void*)g_strips_f32in) || check_nargs("skinny_strips_f32in", nargs, 8)) return NULL;
  if (as_ptr(args[0], &x) || as_ptr(args[1], &wd) || as_ptr(args[2], &out) || as_ptr(args[3], &bias) ||
      as_int(args[4], &M) || as_int(args[5], &N) || as_int(args[6], &K) || as_ptr(args[7], &stream))
    return NULL;
  Py_BEGIN_ALLOW_THREADS
  st = g_strips_f32in(x, wd, out, bias, M, N, K, stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(st);
}

/* mm_t_gemm(x, x_is_f32, w_t, out, out_is_f16, bias, thresh, M, N, K, num_cus, scratch, scratch_bytes,
 * workspace, workspace_bytes, counters, counter_bytes, stream) -> status of g16_mm_t_gemm */
static PyObject* fast_mm_t_gemm(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  void *x, *w, *out, *bias, *scratch, *ws, *cnt, *stream;
  int x_is_f32, out_is_f16, M, N, K, cus, st;
  size_t scratch_bytes, ws_bytes, cnt_bytes;
  double thresh;
  if (check_bound((const void*)g_mm_t_gemm) || check_nargs("mm_t_gemm", nargs, 18)) return NULL;
  if (as_ptr(args[0], &x) || as_int(args[1], &x_is_f32) || as_ptr(args[2], &w) || as_ptr(args[3], &out) ||
      as_int(args[4], &out_is_f16) || as_ptr(args[5], &bias))
    return NULL;
  thresh = PyFloat_AsDouble(args[6]);
  if (thresh == -1.0 && PyErr_Occurred()) return NULL;
  if (as_int(args[7], &M) || as_int(args[8], &N) || as_int(args[9], &K) || as_int(args[10], &cus) ||
      as_ptr(args[11], &scratch) || as_size(args[12], &scratch_bytes) || as_ptr(args[13], &ws) ||
      as_size(args[14], &ws_bytes) || as_ptr(args[15], &cnt) || as_size(args[16], &cnt_bytes) ||
      as_ptr(args[17], &stream))
    return NULL;
  Py_BEGIN_ALLOW_THREADS
  st = g_mm_t_gemm(x, x_is_f32, w, out, out_is_f16, bias, (float)thresh, M, N, K, cus, scratch, scratch_bytes, ws,
                   ws_bytes, cnt, cnt_bytes, stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(st);
}

static PyMethodDef fast_methods[] = {
    {"bind", (PyCFunction)(void (*)(void))fast_bind, METH_FASTCALL,
     "bind(skinny_f32in_addr, mm_t_gemm_addr, skinny_strips_f32in_addr)"},
    {"skinny_strips_f32in", (PyCFunction)(void (*)(void))fast_strips_f32in, METH_FASTCALL,
     "g16_skinny_strips_f32in with fast argument parsing; returns its status"},
    {"skinny_f32in", (PyCFunction)(void (*)(void))fast_skinny_f32in, METH_FASTCALL,
     "g16_skinny_f32in with fast argument parsing; returns its status"},
    {"mm_t_gemm", (PyCFunction)(void (*)(void))fast_mm_t_gemm, METH_FASTCALL,
     "g16_mm_t_gemm with fast argument parsing; returns its status"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef fast_module = {PyModuleDef_HEAD_INIT, "_g16fast", NULL, -1, fast_methods,
                                         NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__g16fast(void) { return PyModule_Create(&fast_module); }
