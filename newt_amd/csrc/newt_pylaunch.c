/*
 * newt_pylaunch.c - the warm-launch path of @newt.jit in C (CPython extension
 * `_newt_launch`).
 *
 * A newt launch from Python must find the specialization its arguments select
 * (dtypes, 16-byte alignment and device of the tensors; ==1, power-of-two
 * divisibility and int32 range of the integers; the constexpr values, launch
 * options and codegen switches), read the parameter values, pack them into
 * the kernel's argument segment and launch. The reference does this in
 * Python on every call (newt/runtime/jit.py:166-223); here the Python path
 * runs once per call signature and registers a plan, and later calls with the
 * same signature run in this file:
 *
 *   run(table, cx_pos, grid, args, kwargs) builds the call's key, looks it up
 *   in `table` (a dict owned by the JIT function) and, on a hit, packs the
 *   arguments and calls newt_launch_packed (include/newt_hip.h) on torch's
 *   current stream. Returns None after a launch (or for an empty grid), the
 *   key (a tuple) on a miss, False when the call has a shape this path does
 *   not handle (the caller then takes the Python path and registers
 *   nothing), or the nonzero status of a failed launch.
 *
 *   make_plan(func, block, argsize, slots) builds a plan: the kernel handle,
 *   the workgroup size, the argument segment's size and, per parameter, the
 *   positional argument it comes from, its kind and its byte offset.
 *
 * The key holds the same facts as the Python signature: positional
 * constexprs and every keyword argument (constexprs and launch options) by
 * type and value, per runtime argument its kind and the facts the code
 * generator specializes on, the current device and the codegen switches.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <dlfcn.h>
#include <stdint.h>
#include <string.h>

typedef int (*launch_packed_fn)(void* function, unsigned gx, unsigned gy, unsigned gz,
                                unsigned block, unsigned lds_bytes, void* stream,
                                const void* argbuf, size_t argsize);

static launch_packed_fn g_launch = NULL;
static PyObject* g_getdev = NULL;     /* torch._C._cuda_getDevice */
static PyObject* g_getstream = NULL;  /* torch._C._cuda_getCurrentRawStream */
static PyObject* g_environ = NULL;    /* os.environ._data */
static PyObject* g_envkeys = NULL;    /* tuple of bytes: the codegen switches */
static PyObject* g_tensor = NULL;     /* torch.Tensor */
static PyObject* s_data_ptr = NULL;
static PyObject* s_get_device = NULL;
static PyObject* s_dtype = NULL;

enum { K_PTR = 0, K_F32 = 1, K_I32 = 2, K_I64 = 3, K_BOOL = 4 };
#define MAX_ARGS 64
#define MAX_SEG 1024

typedef struct {
  int pos, kind, off;
} Slot;

typedef struct {
  void* func;
  unsigned block;
  Py_ssize_t argsize;
  int n;
  Slot slot[MAX_ARGS];
} Plan;

static const char* PLAN_NAME = "newt.launch_plan";

static void plan_free(PyObject* cap) { PyMem_Free(PyCapsule_GetPointer(cap, PLAN_NAME)); }

static PyObject* py_init(PyObject* self, PyObject* args) {
  const char* libpath;
  PyObject *getdev, *getstream, *environ, *envkeys, *tensor;
  if (!PyArg_ParseTuple(args, "sOOO!O!O", &libpath, &getdev, &getstream, &PyDict_Type, &environ,
                        &PyTuple_Type, &envkeys, &tensor))
    return NULL;
  void* h = dlopen(libpath, RTLD_NOW | RTLD_GLOBAL);
  if (!h) return PyErr_Format(PyExc_OSError, "dlopen %s: %s", libpath, dlerror());
  g_launch = (launch_packed_fn)dlsym(h, "newt_launch_packed");
  if (!g_launch) return PyErr_Format(PyExc_OSError, "newt_launch_packed not in %s", libpath);
  Py_XSETREF(g_getdev, Py_NewRef(getdev));
  Py_XSETREF(g_getstream, Py_NewRef(getstream));
  Py_XSETREF(g_environ, Py_NewRef(environ));
  Py_XSETREF(g_envkeys, Py_NewRef(envkeys));
  Py_XSETREF(g_tensor, Py_NewRef(tensor));
  Py_RETURN_NONE;
}

static PyObject* py_make_plan(PyObject* self, PyObject* args) {
  unsigned long long func;
  unsigned block;
  Py_ssize_t argsize;
  PyObject* slots;
  if (!PyArg_ParseTuple(args, "KInO!", &func, &block, &argsize, &PyTuple_Type, &slots))
    return NULL;
  Py_ssize_t n = PyTuple_GET_SIZE(slots);
  if (n > MAX_ARGS || argsize > MAX_SEG || argsize < 0)
    return PyErr_Format(PyExc_ValueError, "launch plan too large (%zd parameters, %zd bytes)",
                        n, argsize);
  Plan* p = (Plan*)PyMem_Calloc(1, sizeof(Plan));
  if (!p) return PyErr_NoMemory();
  p->func = (void*)(uintptr_t)func;
  p->block = block;
  p->argsize = argsize;
  p->n = (int)n;
  for (Py_ssize_t i = 0; i < n; i++) {
    Slot* s = &p->slot[i];
    if (!PyArg_ParseTuple(PyTuple_GET_ITEM(slots, i), "iii", &s->pos, &s->kind, &s->off)) {
      PyMem_Free(p);
      return NULL;
    }
    int width = s->kind == K_BOOL ? 1 : (s->kind == K_F32 || s->kind == K_I32) ? 4 : 8;
    if (s->pos < 0 || s->pos >= MAX_ARGS || s->kind < 0 || s->kind > K_BOOL || s->off < 0 ||
        s->off + width > argsize) {
      PyMem_Free(p);
      return PyErr_Format(PyExc_ValueError, "bad launch plan slot %zd", i);
    }
  }
  PyObject* cap = PyCapsule_New(p, PLAN_NAME, plan_free);
  if (!cap) PyMem_Free(p);
  return cap;
}

/* key bytes: one record per positional argument */
typedef struct {
  unsigned char tag, flags, pad[2];
  int32_t device;
  uint64_t dtype;
} Rec;

static PyObject* call_noargs(PyObject* obj, PyObject* name) {
  return PyObject_VectorcallMethod(name, &obj, 1 | PY_VECTORCALL_ARGUMENTS_OFFSET, NULL);
}

static PyObject* py_run(PyObject* self, PyObject* const* a, Py_ssize_t na) {
  if (na != 5) return PyErr_Format(PyExc_TypeError, "run() takes 5 arguments");
  PyObject *table = a[0], *cx = a[1], *grid = a[2], *args = a[3], *kwargs = a[4];
  if (!g_launch) return PyErr_Format(PyExc_RuntimeError, "_newt_launch.init() was not called");
  if (!PyDict_Check(table) || !PyTuple_Check(cx) || !PyTuple_Check(args) || !PyDict_Check(kwargs))
    return PyErr_Format(PyExc_TypeError, "run(table, cx_pos, grid, args, kwargs)");
  Py_ssize_t nargs = PyTuple_GET_SIZE(args), ncx = PyTuple_GET_SIZE(cx);
  if (nargs > MAX_ARGS) Py_RETURN_FALSE;

  /* the launch grid: an int or a tuple of 1-3 ints (a callable grid takes the
     Python path) */
  long g[3] = {1, 1, 1};
  if (PyLong_CheckExact(grid)) {
    g[0] = PyLong_AsLong(grid);
  } else if (PyTuple_CheckExact(grid) && PyTuple_GET_SIZE(grid) >= 1 &&
             PyTuple_GET_SIZE(grid) <= 3) {
    for (Py_ssize_t i = 0; i < PyTuple_GET_SIZE(grid); i++) {
      PyObject* v = PyTuple_GET_ITEM(grid, i);
      if (!PyLong_CheckExact(v)) Py_RETURN_FALSE;
      g[i] = PyLong_AsLong(v);
    }
  } else {
    Py_RETURN_FALSE;
  }
  if (PyErr_Occurred()) return NULL;
  for (int i = 0; i < 3; i++)
    if (g[i] > 0xFFFFFFFFL) Py_RETURN_FALSE;

  PyObject* devobj = PyObject_CallNoArgs(g_getdev);
  if (!devobj) return NULL;
  long device = PyLong_AsLong(devobj);
  if (device == -1 && PyErr_Occurred()) {
    Py_DECREF(devobj);
    return NULL;
  }

  Rec rec[MAX_ARGS + 1];
  uint64_t ptrs[MAX_ARGS];
  memset(rec, 0, sizeof(Rec) * (nargs + 1));
  rec[nargs].tag = 'D';
  rec[nargs].device = (int32_t)device;
  PyObject* extra = PyList_New(0);
  if (!extra) {
    Py_DECREF(devobj);
    return NULL;
  }
  PyObject* result = NULL;
  PyObject* key = NULL;
  for (Py_ssize_t i = 0; i < nargs; i++) {
    PyObject* v = PyTuple_GET_ITEM(args, i);
    Rec* r = &rec[i];
    if (i < ncx && PyTuple_GET_ITEM(cx, i) == Py_True) {
      r->tag = 'C';
      PyObject* t = PyTuple_Pack(2, (PyObject*)Py_TYPE(v), v);
      if (!t || PyList_Append(extra, t) < 0) {
        Py_XDECREF(t);
        goto done;
      }
      Py_DECREF(t);
    } else if (PyBool_Check(v)) {
      r->tag = 'b';
    } else if (PyLong_CheckExact(v)) {
      int overflow = 0;
      long long x = PyLong_AsLongLongAndOverflow(v, &overflow);
      if (overflow) {
        result = Py_NewRef(Py_False);
        goto done;
      }
      if (x == -1 && PyErr_Occurred()) goto done;
      unsigned long long m = x < 0 ? 0ULL - (unsigned long long)x : (unsigned long long)x;
      unsigned d = m == 0 ? 16 : (unsigned)(m & (0ULL - m));
      if (d > 16) d = 16;
      r->tag = 'i';
      r->flags = (unsigned char)(d | ((x == 1) << 5) | ((x >= INT32_MIN && x <= INT32_MAX) << 6));
    } else if (PyFloat_CheckExact(v)) {
      r->tag = 'f';
    } else if (PyObject_TypeCheck(v, (PyTypeObject*)g_tensor)) {
      PyObject* dt = PyObject_GetAttr(v, s_dtype);
      if (!dt) goto done;
      r->dtype = (uint64_t)(uintptr_t)dt; /* dtypes are module-level singletons */
      Py_DECREF(dt);
      PyObject* p = call_noargs(v, s_data_ptr);
      if (!p) goto done;
      ptrs[i] = (uint64_t)PyLong_AsUnsignedLongLong(p);
      Py_DECREF(p);
      if (PyErr_Occurred()) goto done;
      PyObject* dv = call_noargs(v, s_get_device);
      if (!dv) goto done;
      r->device = (int32_t)PyLong_AsLong(dv);
      Py_DECREF(dv);
      if (PyErr_Occurred()) goto done;
      r->tag = 't';
      r->flags = (ptrs[i] & 15) == 0;
    } else {
      result = Py_NewRef(Py_False);
      goto done;
    }
  }
  {
    PyObject *k, *v;
    Py_ssize_t pos = 0;
    while (PyDict_Next(kwargs, &pos, &k, &v)) {
      PyObject* t = PyTuple_Pack(3, k, (PyObject*)Py_TYPE(v), v);
      if (!t || PyList_Append(extra, t) < 0) {
        Py_XDECREF(t);
        goto done;
      }
      Py_DECREF(t);
    }
  }
  {
    Py_ssize_t ne = PyTuple_GET_SIZE(g_envkeys);
    PyObject* env = PyTuple_New(ne);
    if (!env) goto done;
    for (Py_ssize_t i = 0; i < ne; i++) {
      PyObject* val = PyDict_GetItemWithError(g_environ, PyTuple_GET_ITEM(g_envkeys, i));
      if (!val && PyErr_Occurred()) {
        Py_DECREF(env);
        goto done;
      }
      PyTuple_SET_ITEM(env, i, Py_NewRef(val ? val : Py_None));
    }
    PyObject* bytes = PyBytes_FromStringAndSize((const char*)rec, sizeof(Rec) * (nargs + 1));
    PyObject* ex = bytes ? PyList_AsTuple(extra) : NULL;
    key = (bytes && ex) ? PyTuple_Pack(3, bytes, env, ex) : NULL;
    Py_XDECREF(bytes);
    Py_XDECREF(ex);
    Py_DECREF(env);
    if (!key) goto done;
  }
  {
    PyObject* cap = PyDict_GetItemWithError(table, key); /* borrowed */
    if (!cap) {
      if (!PyErr_Occurred()) result = Py_NewRef(key);
      goto done;
    }
    Plan* p = (Plan*)PyCapsule_GetPointer(cap, PLAN_NAME);
    if (!p) goto done;
    if (g[0] <= 0 || g[1] <= 0 || g[2] <= 0) { /* empty grid: no-op */
      result = Py_NewRef(Py_None);
      goto done;
    }
    unsigned char seg[MAX_SEG] __attribute__((aligned(16)));
    memset(seg, 0, (size_t)p->argsize);
    for (int j = 0; j < p->n; j++) {
      const Slot* s = &p->slot[j];
      if (s->pos >= nargs) {
        result = Py_NewRef(Py_False);
        goto done;
      }
      PyObject* v = PyTuple_GET_ITEM(args, s->pos);
      switch (s->kind) {
        case K_PTR:
          if (rec[s->pos].tag != 't') {
            result = Py_NewRef(Py_False);
            goto done;
          }
          memcpy(seg + s->off, &ptrs[s->pos], 8);
          break;
        case K_F32: {
          double d = PyFloat_AsDouble(v);
          if (d == -1.0 && PyErr_Occurred()) goto done;
          float f = (float)d;
          memcpy(seg + s->off, &f, 4);
          break;
        }
        case K_I32: {
          long x = PyLong_AsLong(v);
          if (x == -1 && PyErr_Occurred()) goto done;
          int32_t y = (int32_t)x;
          memcpy(seg + s->off, &y, 4);
          break;
        }
        case K_I64: {
          long long x = PyLong_AsLongLong(v);
          if (x == -1 && PyErr_Occurred()) goto done;
          memcpy(seg + s->off, &x, 8);
          break;
        }
        default: {
          int b = PyObject_IsTrue(v);
          if (b < 0) goto done;
          seg[s->off] = (unsigned char)b;
        }
      }
    }
    PyObject* st = PyObject_CallOneArg(g_getstream, devobj);
    if (!st) goto done;
    void* stream = PyLong_AsVoidPtr(st);
    Py_DECREF(st);
    if (PyErr_Occurred()) goto done;
    int rc = g_launch(p->func, (unsigned)g[0], (unsigned)g[1], (unsigned)g[2], p->block, 0,
                      stream, seg, (size_t)p->argsize);
    result = rc ? PyLong_FromLong(rc) : Py_NewRef(Py_None);
  }
done:
  Py_XDECREF(key);
  Py_DECREF(extra);
  Py_DECREF(devobj);
  return result;
}

static PyMethodDef methods[] = {
    {"init", py_init, METH_VARARGS,
     "init(libnewt_hip_path, get_device, get_raw_stream, environ_data, env_keys, tensor_type)"},
    {"make_plan", py_make_plan, METH_VARARGS, "make_plan(func, block, argsize, slots)"},
    {"run", (PyCFunction)(void (*)(void))py_run, METH_FASTCALL,
     "run(table, cx_pos, grid, args, kwargs) -> None | key | False | status"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_newt_launch",
                                    "Warm-launch path of @newt.jit kernels.", -1, methods};

PyMODINIT_FUNC PyInit__newt_launch(void) {
  s_data_ptr = PyUnicode_InternFromString("data_ptr");
  s_get_device = PyUnicode_InternFromString("get_device");
  s_dtype = PyUnicode_InternFromString("dtype");
  if (!s_data_ptr || !s_get_device || !s_dtype) return NULL;
  return PyModule_Create(&module);
}
