/*
 * _kvhfast: the per-step entry points of libkvhip (include/kvhip.h) as CPython functions.
 *
 * At decode sizes the host side of a call is of the order of the kernels themselves, and
 * ctypes spends several microseconds converting the ~30 arguments of kvh_paged_attention.
 * These wrappers take the same arguments as plain Python ints and floats (pointers as ints,
 * each stride array as three ints) with METH_FASTCALL, convert them in C and call the C ABI;
 * they return its status code. No torch types cross this layer either. The entry points
 * are looked up (dlsym) in the library the ctypes binding opened, handed over by bind(), so
 * both bindings always call the same library.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <dlfcn.h>
#include <stdint.h>

#include "kvhip.h"

static __typeof__(kvh_paged_attention)* f_paged_attention;
static __typeof__(kvh_paged_attention_fp8)* f_paged_attention_fp8;
static __typeof__(kvh_reshape_and_cache)* f_reshape_and_cache;
static __typeof__(kvh_reshape_and_cache_fp8)* f_reshape_and_cache_fp8;
static __typeof__(kvh_rope_and_cache)* f_rope_and_cache;
static __typeof__(kvh_rope_and_cache_fp8)* f_rope_and_cache_fp8;

/* bind(handle): resolve the entry points in the dlopen handle of the loaded libkvhip */
static PyObject* bind(PyObject* self, PyObject* arg) {
  (void)self;
  void* h = PyLong_AsVoidPtr(arg);
  if (h == NULL) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_ValueError, "bind: NULL library handle");
    return NULL;
  }
#define SYM(var, name)                                                             \
  var = (__typeof__(var))dlsym(h, name);                                           \
  if (var == NULL) {                                                               \
    PyErr_Format(PyExc_RuntimeError, "bind: libkvhip does not export %s", name);   \
    return NULL;                                                                   \
  }
  SYM(f_paged_attention, "kvh_paged_attention")
  SYM(f_paged_attention_fp8, "kvh_paged_attention_fp8")
  SYM(f_reshape_and_cache, "kvh_reshape_and_cache")
  SYM(f_reshape_and_cache_fp8, "kvh_reshape_and_cache_fp8")
  SYM(f_rope_and_cache, "kvh_rope_and_cache")
  SYM(f_rope_and_cache_fp8, "kvh_rope_and_cache_fp8")
#undef SYM
  Py_RETURN_NONE;
}

static int as_i64(PyObject* o, int64_t* v) {
  *v = (int64_t)PyLong_AsLongLong(o);
  return !(*v == -1 && PyErr_Occurred());
}

static int as_ptr(PyObject* o, void** v) {
  if (o == Py_None) {
    *v = NULL;
    return 1;
  }
  *v = PyLong_AsVoidPtr(o);
  return !(*v == NULL && PyErr_Occurred());
}

static int as_f32(PyObject* o, float* v) {
  const double d = PyFloat_AsDouble(o);
  *v = (float)d;
  return !(d == -1.0 && PyErr_Occurred());
}

#define ARG_I64(i, name) \
  int64_t name;          \
  if (!as_i64(args[i], &name)) return NULL;
#define ARG_PTR(i, name) \
  void* name;            \
  if (!as_ptr(args[i], &name)) return NULL;
#define ARG_F32(i, name) \
  float name;            \
  if (!as_f32(args[i], &name)) return NULL;
#define ARG_STRIDES(i, name) \
  int64_t name[3];           \
  if (!as_i64(args[i], &name[0]) || !as_i64(args[i + 1], &name[1]) || !as_i64(args[i + 2], &name[2])) return NULL;

static int check_nargs(Py_ssize_t nargs, Py_ssize_t want, const char* fn) {
  if (f_paged_attention == NULL) {
    PyErr_SetString(PyExc_RuntimeError, "_kvhfast: bind() the loaded libkvhip first");
    return 0;
  }
  if (nargs == want) return 1;
  PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", fn, want, nargs);
  return 0;
}

/* paged_attention(q, q_ts, q_hs, kc, kcs0, kcs1, kcs2, vc, vcs0, vcs1, vcs2, num_blocks, out, o_ts, o_hs,
 *                 bt, bt_rs, width, seq_lens, qsl, T, B, H, Hkv, D, BS, max_q, scale, dtype, ws, ws_bytes,
 *                 stream) -> status  (kvh_paged_attention) */
static PyObject* paged_attention(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (!check_nargs(nargs, 32, "paged_attention")) return NULL;
  ARG_PTR(0, q) ARG_I64(1, q_ts) ARG_I64(2, q_hs) ARG_PTR(3, kc) ARG_STRIDES(4, kcs) ARG_PTR(7, vc)
  ARG_STRIDES(8, vcs) ARG_I64(11, nb) ARG_PTR(12, out) ARG_I64(13, o_ts) ARG_I64(14, o_hs) ARG_PTR(15, bt)
  ARG_I64(16, bt_rs) ARG_I64(17, width) ARG_PTR(18, sl) ARG_PTR(19, qsl) ARG_I64(20, T) ARG_I64(21, B)
  ARG_I64(22, H) ARG_I64(23, Hkv) ARG_I64(24, D) ARG_I64(25, BS) ARG_I64(26, max_q) ARG_F32(27, scale)
  ARG_I64(28, dtype) ARG_PTR(29, ws) ARG_I64(30, ws_bytes) ARG_PTR(31, stream)
  const int st = f_paged_attention(q, q_ts, q_hs, kc, kcs, vc, vcs, nb, out, o_ts, o_hs, (const int64_t*)bt, bt_rs,
                                     (int32_t)width, (const int64_t*)sl, (const int64_t*)qsl, T, (int32_t)B,
                                     (int32_t)H, (int32_t)Hkv, (int32_t)D, (int32_t)BS, (int32_t)max_q, scale,
                                     (int32_t)dtype, ws, (size_t)ws_bytes, stream);
  return PyLong_FromLong(st);
}

/* paged_attention_fp8(..., scale, k_scale, v_scale, dtype, ws, ws_bytes, stream): the same with the two
 * E4M3 scales after `scale` (kvh_paged_attention_fp8) */
static PyObject* paged_attention_fp8(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (!check_nargs(nargs, 34, "paged_attention_fp8")) return NULL;
  ARG_PTR(0, q) ARG_I64(1, q_ts) ARG_I64(2, q_hs) ARG_PTR(3, kc) ARG_STRIDES(4, kcs) ARG_PTR(7, vc)
  ARG_STRIDES(8, vcs) ARG_I64(11, nb) ARG_PTR(12, out) ARG_I64(13, o_ts) ARG_I64(14, o_hs) ARG_PTR(15, bt)
  ARG_I64(16, bt_rs) ARG_I64(17, width) ARG_PTR(18, sl) ARG_PTR(19, qsl) ARG_I64(20, T) ARG_I64(21, B)
  ARG_I64(22, H) ARG_I64(23, Hkv) ARG_I64(24, D) ARG_I64(25, BS) ARG_I64(26, max_q) ARG_F32(27, scale)
  ARG_F32(28, k_scale) ARG_F32(29, v_scale) ARG_I64(30, dtype) ARG_PTR(31, ws) ARG_I64(32, ws_bytes)
  ARG_PTR(33, stream)
  const int st = f_paged_attention_fp8(q, q_ts, q_hs, kc, kcs, vc, vcs, nb, out, o_ts, o_hs, (const int64_t*)bt,
                                         bt_rs, (int32_t)width, (const int64_t*)sl, (const int64_t*)qsl, T,
                                         (int32_t)B, (int32_t)H, (int32_t)Hkv, (int32_t)D, (int32_t)BS,
                                         (int32_t)max_q, scale, k_scale, v_scale, (int32_t)dtype, ws,
                                         (size_t)ws_bytes, stream);
  return PyLong_FromLong(st);
}

/* reshape_and_cache(k, k_ts, k_hs, v, v_ts, v_hs, kc, kcs0, kcs1, kcs2, vc, vcs0, vcs1, vcs2, slots, T,
 *                   num_blocks, Hkv, D, BS, dtype, stream) -> status  (kvh_reshape_and_cache) */
static PyObject* reshape_and_cache(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (!check_nargs(nargs, 22, "reshape_and_cache")) return NULL;
  ARG_PTR(0, k) ARG_I64(1, k_ts) ARG_I64(2, k_hs) ARG_PTR(3, v) ARG_I64(4, v_ts) ARG_I64(5, v_hs)
  ARG_PTR(6, kc) ARG_STRIDES(7, kcs) ARG_PTR(10, vc) ARG_STRIDES(11, vcs) ARG_PTR(14, slots) ARG_I64(15, T)
  ARG_I64(16, nb) ARG_I64(17, Hkv) ARG_I64(18, D) ARG_I64(19, BS) ARG_I64(20, dtype) ARG_PTR(21, stream)
  const int st = f_reshape_and_cache(k, k_ts, k_hs, v, v_ts, v_hs, kc, kcs, vc, vcs, (const int64_t*)slots, T, nb,
                                       (int32_t)Hkv, (int32_t)D, (int32_t)BS, (int32_t)dtype, stream);
  return PyLong_FromLong(st);
}

/* reshape_and_cache_fp8(..., dtype, k_scale, v_scale, stream) (kvh_reshape_and_cache_fp8) */
static PyObject* reshape_and_cache_fp8(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (!check_nargs(nargs, 24, "reshape_and_cache_fp8")) return NULL;
  ARG_PTR(0, k) ARG_I64(1, k_ts) ARG_I64(2, k_hs) ARG_PTR(3, v) ARG_I64(4, v_ts) ARG_I64(5, v_hs)
  ARG_PTR(6, kc) ARG_STRIDES(7, kcs) ARG_PTR(10, vc) ARG_STRIDES(11, vcs) ARG_PTR(14, slots) ARG_I64(15, T)
  ARG_I64(16, nb) ARG_I64(17, Hkv) ARG_I64(18, D) ARG_I64(19, BS) ARG_I64(20, dtype) ARG_F32(21, k_scale)
  ARG_F32(22, v_scale) ARG_PTR(23, stream)
  const int st = f_reshape_and_cache_fp8(k, k_ts, k_hs, v, v_ts, v_hs, kc, kcs, vc, vcs, (const int64_t*)slots, T,
                                           nb, (int32_t)Hkv, (int32_t)D, (int32_t)BS, (int32_t)dtype, k_scale,
                                           v_scale, stream);
  return PyLong_FromLong(st);
}

/* rope_and_cache(qkv, qkv_ts, positions, cos, sin, max_pos, q_out, q_ts, q_hs, kc, kcs0, kcs1, kcs2, vc,
 *                vcs0, vcs1, vcs2, slots, T, num_blocks, H, Hkv, D, BS, dtype, kv_fp8, k_scale, v_scale,
 *                stream) -> status  (kvh_rope_and_cache, or kvh_rope_and_cache_fp8 when kv_fp8) */
static PyObject* rope_and_cache(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (!check_nargs(nargs, 29, "rope_and_cache")) return NULL;
  ARG_PTR(0, qkv) ARG_I64(1, qkv_ts) ARG_PTR(2, pos) ARG_PTR(3, cs) ARG_PTR(4, sn) ARG_I64(5, max_pos)
  ARG_PTR(6, q_out) ARG_I64(7, q_ts) ARG_I64(8, q_hs) ARG_PTR(9, kc) ARG_STRIDES(10, kcs) ARG_PTR(13, vc)
  ARG_STRIDES(14, vcs) ARG_PTR(17, slots) ARG_I64(18, T) ARG_I64(19, nb) ARG_I64(20, H) ARG_I64(21, Hkv)
  ARG_I64(22, D) ARG_I64(23, BS) ARG_I64(24, dtype) ARG_I64(25, fp8) ARG_F32(26, k_scale) ARG_F32(27, v_scale)
  ARG_PTR(28, stream)
  int st;
  if (fp8)
    st = f_rope_and_cache_fp8(qkv, qkv_ts, (const int64_t*)pos, (const float*)cs, (const float*)sn, max_pos,
                                q_out, q_ts, q_hs, kc, kcs, vc, vcs, (const int64_t*)slots, T, nb, (int32_t)H,
                                (int32_t)Hkv, (int32_t)D, (int32_t)BS, (int32_t)dtype, k_scale, v_scale, stream);
  else
    st = f_rope_and_cache(qkv, qkv_ts, (const int64_t*)pos, (const float*)cs, (const float*)sn, max_pos, q_out,
                            q_ts, q_hs, kc, kcs, vc, vcs, (const int64_t*)slots, T, nb, (int32_t)H, (int32_t)Hkv,
                            (int32_t)D, (int32_t)BS, (int32_t)dtype, stream);
  return PyLong_FromLong(st);
}

static PyMethodDef methods[] = {
    {"bind", bind, METH_O, "resolve the entry points in a dlopen handle of libkvhip"},
    {"paged_attention", (PyCFunction)(void (*)(void))paged_attention, METH_FASTCALL, "kvh_paged_attention"},
    {"paged_attention_fp8", (PyCFunction)(void (*)(void))paged_attention_fp8, METH_FASTCALL,
     "kvh_paged_attention_fp8"},
    {"reshape_and_cache", (PyCFunction)(void (*)(void))reshape_and_cache, METH_FASTCALL, "kvh_reshape_and_cache"},
    {"reshape_and_cache_fp8", (PyCFunction)(void (*)(void))reshape_and_cache_fp8, METH_FASTCALL,
     "kvh_reshape_and_cache_fp8"},
    {"rope_and_cache", (PyCFunction)(void (*)(void))rope_and_cache, METH_FASTCALL,
     "kvh_rope_and_cache / kvh_rope_and_cache_fp8"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_kvhfast", "libkvhip's per-step entry points", -1,
                                    methods};

PyMODINIT_FUNC PyInit__kvhfast(void) { return PyModule_Create(&module); }
