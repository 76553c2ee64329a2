/*
 * CPython binding over the C ABI (include/nibblegemm_amd.h).
 *
 * Every function takes plain integers: device pointers as Python ints (from
 * torch.Tensor.data_ptr()), shapes, and the HIP stream handle.  It forwards to
 * the library and returns the integer status; the Python layer
 * (nibblegemm_amd/ops.py) turns a non-zero status into RuntimeError with
 * last_error().  Built as METH_FASTCALL so per-call overhead stays well under
 * a microsecond next to ~4 us kernels.  No torch headers, no torch types.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include "../../include/nibblegemm_amd.h"

static int take_i64(PyObject* o, long long* out) {
  *out = PyLong_AsLongLong(o);
  return !(*out == -1 && PyErr_Occurred());
}

static int take_ptr(PyObject* o, void** out) {
  if (o == Py_None) {
    *out = NULL;
    return 1;
  }
  *out = PyLong_AsVoidPtr(o);
  return !(*out == NULL && PyErr_Occurred());
}

static int nargs_is(Py_ssize_t n, Py_ssize_t want, const char* name) {
  if (n != want) {
    PyErr_Format(PyExc_TypeError, "%s expects %zd arguments, got %zd", name, want, n);
    return 0;
  }
  return 1;
}

/* gemv(X, xr, xc, Wq, wr, wc, S, sr, sc, g, version, splits, threads, Y, ws, ws_bytes, stream) */
static PyObject* py_gemv(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 17, "gemv")) return NULL;
  void *X, *Wq, *S, *Y, *ws, *stream;
  long long xr, xc, wr, wc, sr, sc, g, ver, spl, thr, wsb;
  if (!take_ptr(a[0], &X) || !take_i64(a[1], &xr) || !take_i64(a[2], &xc) ||
      !take_ptr(a[3], &Wq) || !take_i64(a[4], &wr) || !take_i64(a[5], &wc) ||
      !take_ptr(a[6], &S) || !take_i64(a[7], &sr) || !take_i64(a[8], &sc) ||
      !take_i64(a[9], &g) || !take_i64(a[10], &ver) || !take_i64(a[11], &spl) ||
      !take_i64(a[12], &thr) || !take_ptr(a[13], &Y) || !take_ptr(a[14], &ws) ||
      !take_i64(a[15], &wsb) || !take_ptr(a[16], &stream))
    return NULL;
  int rc = nibble_gemv_w4a16(X, xr, xc, Wq, wr, wc, S, sr, sc, g, ver, spl, thr, Y, ws,
                             (size_t)(wsb < 0 ? 0 : wsb), stream);
  return PyLong_FromLong(rc);
}

/* gemv_workspace_bytes(M, K, N, g, version, splits, threads, stream) */
static PyObject* py_gemv_ws(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 8, "gemv_workspace_bytes")) return NULL;
  long long M, K, N, g, ver, spl, thr;
  void* stream;
  if (!take_i64(a[0], &M) || !take_i64(a[1], &K) || !take_i64(a[2], &N) || !take_i64(a[3], &g) ||
      !take_i64(a[4], &ver) || !take_i64(a[5], &spl) || !take_i64(a[6], &thr) ||
      !take_ptr(a[7], &stream))
    return NULL;
  size_t ws = nibble_gemv_workspace_bytes(M, K, N, g, ver, spl, thr, stream);
  size_t cb = nibble_gemv_counter_bytes(M, K, N, g, ver, spl, thr, stream);
  return Py_BuildValue("(nn)", (Py_ssize_t)ws, (Py_ssize_t)cb);
}

/* gemm(X, xr, xc, Wq, wr, wc, S, sr, sc, g, version, Y, ws, ws_bytes, stream) */
static PyObject* py_gemm(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 15, "gemm")) return NULL;
  void *X, *Wq, *S, *Y, *ws, *stream;
  long long xr, xc, wr, wc, sr, sc, g, ver, wsb;
  if (!take_ptr(a[0], &X) || !take_i64(a[1], &xr) || !take_i64(a[2], &xc) ||
      !take_ptr(a[3], &Wq) || !take_i64(a[4], &wr) || !take_i64(a[5], &wc) ||
      !take_ptr(a[6], &S) || !take_i64(a[7], &sr) || !take_i64(a[8], &sc) ||
      !take_i64(a[9], &g) || !take_i64(a[10], &ver) || !take_ptr(a[11], &Y) ||
      !take_ptr(a[12], &ws) || !take_i64(a[13], &wsb) || !take_ptr(a[14], &stream))
    return NULL;
  int rc = nibble_gemm_w4a16(X, xr, xc, Wq, wr, wc, S, sr, sc, g, ver, Y, ws,
                             (size_t)(wsb < 0 ? 0 : wsb), stream);
  return PyLong_FromLong(rc);
}

/* gemm_workspace_bytes(M, K, N, g, version, stream) */
static PyObject* py_gemm_ws(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 6, "gemm_workspace_bytes")) return NULL;
  long long M, K, N, g, ver;
  void* stream;
  if (!take_i64(a[0], &M) || !take_i64(a[1], &K) || !take_i64(a[2], &N) || !take_i64(a[3], &g) ||
      !take_i64(a[4], &ver) || !take_ptr(a[5], &stream))
    return NULL;
  size_t ws = nibble_gemm_workspace_bytes(M, K, N, g, ver, stream);
  size_t cb = nibble_gemm_counter_bytes(M, K, N, g, ver, stream);
  return Py_BuildValue("(nn)", (Py_ssize_t)ws, (Py_ssize_t)cb);
}

/* matmul_fused(X, xr, xc, Wq, wr, wc, S, sr, sc, g, epilogue, bias, norm_w, norm_eps, Y, ws,
 *              ws_bytes, stream) */
static PyObject* py_fused(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 18, "matmul_fused")) return NULL;
  void *X, *Wq, *S, *bias, *norm, *Y, *ws, *stream;
  long long xr, xc, wr, wc, sr, sc, g, ep, wsb;
  double eps = PyFloat_AsDouble(a[13]);
  if (eps == -1.0 && PyErr_Occurred()) return NULL;
  if (!take_ptr(a[0], &X) || !take_i64(a[1], &xr) || !take_i64(a[2], &xc) ||
      !take_ptr(a[3], &Wq) || !take_i64(a[4], &wr) || !take_i64(a[5], &wc) ||
      !take_ptr(a[6], &S) || !take_i64(a[7], &sr) || !take_i64(a[8], &sc) ||
      !take_i64(a[9], &g) || !take_i64(a[10], &ep) || !take_ptr(a[11], &bias) ||
      !take_ptr(a[12], &norm) || !take_ptr(a[14], &Y) || !take_ptr(a[15], &ws) ||
      !take_i64(a[16], &wsb) || !take_ptr(a[17], &stream))
    return NULL;
  int rc = nibble_matmul_w4a16_fused(X, xr, xc, Wq, wr, wc, S, sr, sc, g, ep, bias, norm,
                                     (float)eps, Y, ws, (size_t)(wsb < 0 ? 0 : wsb), stream);
  return PyLong_FromLong(rc);
}

/* matmul_fused_workspace_bytes(M, K, N, g, stream) */
static PyObject* py_fused_ws(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 5, "matmul_fused_workspace_bytes")) return NULL;
  long long M, K, N, g;
  void* stream;
  if (!take_i64(a[0], &M) || !take_i64(a[1], &K) || !take_i64(a[2], &N) || !take_i64(a[3], &g) ||
      !take_ptr(a[4], &stream))
    return NULL;
  size_t ws = nibble_matmul_fused_workspace_bytes(M, K, N, g, stream);
  size_t cb = nibble_matmul_fused_counter_bytes(M, K, N, g, stream);
  return Py_BuildValue("(nn)", (Py_ssize_t)ws, (Py_ssize_t)cb);
}

/* gemm_streams(M, K, N, g) */
static PyObject* py_gemm_streams(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 4, "gemm_streams")) return NULL;
  long long M, K, N, g;
  if (!take_i64(a[0], &M) || !take_i64(a[1], &K) || !take_i64(a[2], &N) || !take_i64(a[3], &g))
    return NULL;
  return PyBool_FromLong(nibble_gemm_streams(M, K, N, g));
}

/* strip_major_cols(K, N, g) */
static PyObject* py_sm_cols(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 3, "strip_major_cols")) return NULL;
  long long K, N, g;
  if (!take_i64(a[0], &K) || !take_i64(a[1], &N) || !take_i64(a[2], &g)) return NULL;
  return PyLong_FromLongLong((long long)nibble_strip_major_cols(K, N, g));
}

/* gemv_timeline(stamps_ptr, bytes) */
static PyObject* py_gemv_timeline(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 2, "gemv_timeline")) return NULL;
  void* stamps;
  long long bytes;
  if (!take_ptr(a[0], &stamps) || !take_i64(a[1], &bytes)) return NULL;
  return PyLong_FromLong(nibble_gemv_timeline(stamps, bytes));
}

/* chain_strip_cols(K, N, g, M) */
static PyObject* py_chain_cols(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 4, "chain_strip_cols")) return NULL;
  long long K, N, g, M;
  if (!take_i64(a[0], &K) || !take_i64(a[1], &N) || !take_i64(a[2], &g) || !take_i64(a[3], &M))
    return NULL;
  return PyLong_FromLongLong((long long)nibble_chain_strip_cols(K, N, g, M));
}

/* pack_strip_major(Wq, wr, wc, S, sr, sc, g, strip_cols, Wt, St, stream) */
static PyObject* py_sm_pack(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 11, "pack_strip_major")) return NULL;
  void *Wq, *S, *Wt, *St, *stream;
  long long wr, wc, sr, sc, g, sw;
  if (!take_ptr(a[0], &Wq) || !take_i64(a[1], &wr) || !take_i64(a[2], &wc) ||
      !take_ptr(a[3], &S) || !take_i64(a[4], &sr) || !take_i64(a[5], &sc) ||
      !take_i64(a[6], &g) || !take_i64(a[7], &sw) || !take_ptr(a[8], &Wt) ||
      !take_ptr(a[9], &St) || !take_ptr(a[10], &stream))
    return NULL;
  return PyLong_FromLong(nibble_pack_strip_major(Wq, wr, wc, S, sr, sc, g, sw, Wt, St, stream));
}

/* gemv_strip_major(X, xr, xc, Wt, St, K, N, g, strip_cols, epilogue, bias, norm_w, norm_eps, Y,
 *                  stream) */
static PyObject* py_sm_gemv(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 15, "gemv_strip_major")) return NULL;
  void *X, *Wt, *St, *bias, *norm, *Y, *stream;
  long long xr, xc, K, N, g, sw, ep;
  double eps = PyFloat_AsDouble(a[12]);
  if (eps == -1.0 && PyErr_Occurred()) return NULL;
  if (!take_ptr(a[0], &X) || !take_i64(a[1], &xr) || !take_i64(a[2], &xc) ||
      !take_ptr(a[3], &Wt) || !take_ptr(a[4], &St) || !take_i64(a[5], &K) ||
      !take_i64(a[6], &N) || !take_i64(a[7], &g) || !take_i64(a[8], &sw) ||
      !take_i64(a[9], &ep) || !take_ptr(a[10], &bias) || !take_ptr(a[11], &norm) ||
      !take_ptr(a[13], &Y) || !take_ptr(a[14], &stream))
    return NULL;
  return PyLong_FromLong(nibble_gemv_w4a16_strip_major(X, xr, xc, Wt, St, K, N, g, sw, ep, bias,
                                                       norm, (float)eps, Y, stream));
}

/* rmsnorm(X, rows, cols, W, eps, Y, stream) */
static PyObject* py_rmsnorm(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 7, "rmsnorm")) return NULL;
  void *X, *W, *Y, *stream;
  long long rows, cols;
  double eps = PyFloat_AsDouble(a[4]);
  if (eps == -1.0 && PyErr_Occurred()) return NULL;
  if (!take_ptr(a[0], &X) || !take_i64(a[1], &rows) || !take_i64(a[2], &cols) ||
      !take_ptr(a[3], &W) || !take_ptr(a[5], &Y) || !take_ptr(a[6], &stream))
    return NULL;
  return PyLong_FromLong(nibble_rmsnorm_f16(X, rows, cols, W, (float)eps, Y, stream));
}

/* attention(QKV, n_heads, n_kv, head_dim, Kc, Vc, max_seq, pos, cos, sin, Out, ws, ws_bytes,
 * stream) */
static PyObject* py_attention(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 14, "attention")) return NULL;
  void *qkv, *kc, *vc, *rc, *rs, *out, *ws, *stream;
  long long nh, nkv, hd, ms, pos, wsb;
  if (!take_ptr(a[0], &qkv) || !take_i64(a[1], &nh) || !take_i64(a[2], &nkv) ||
      !take_i64(a[3], &hd) || !take_ptr(a[4], &kc) || !take_ptr(a[5], &vc) ||
      !take_i64(a[6], &ms) || !take_i64(a[7], &pos) || !take_ptr(a[8], &rc) ||
      !take_ptr(a[9], &rs) || !take_ptr(a[10], &out) || !take_ptr(a[11], &ws) ||
      !take_i64(a[12], &wsb) || !take_ptr(a[13], &stream))
    return NULL;
  int rc_ = nibble_attention_decode_f16(qkv, nh, nkv, hd, kc, vc, ms, pos, rc, rs, out, ws,
                                        (size_t)(wsb < 0 ? 0 : wsb), stream);
  return PyLong_FromLong(rc_);
}

/* attention_workspace_bytes(n_heads, n_kv, head_dim, max_seq, pos, stream) */
static PyObject* py_attention_ws(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 6, "attention_workspace_bytes")) return NULL;
  long long nh, nkv, hd, ms, pos;
  void* stream;
  if (!take_i64(a[0], &nh) || !take_i64(a[1], &nkv) || !take_i64(a[2], &hd) ||
      !take_i64(a[3], &ms) || !take_i64(a[4], &pos) || !take_ptr(a[5], &stream))
    return NULL;
  size_t ws = nibble_attention_decode_workspace_bytes(nh, nkv, hd, ms, pos, stream);
  size_t cb = nibble_attention_decode_counter_bytes(nh, nkv, hd, ms, pos, stream);
  return Py_BuildValue("(nn)", (Py_ssize_t)ws, (Py_ssize_t)cb);
}

/* dequant(Wq, wr, wc, S, sr, sc, g, fast, W, stream) */
static PyObject* py_dequant(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 10, "dequant")) return NULL;
  void *Wq, *S, *W, *stream;
  long long wr, wc, sr, sc, g, fast;
  if (!take_ptr(a[0], &Wq) || !take_i64(a[1], &wr) || !take_i64(a[2], &wc) ||
      !take_ptr(a[3], &S) || !take_i64(a[4], &sr) || !take_i64(a[5], &sc) ||
      !take_i64(a[6], &g) || !take_i64(a[7], &fast) || !take_ptr(a[8], &W) ||
      !take_ptr(a[9], &stream))
    return NULL;
  int rc = nibble_dequant_w4(Wq, wr, wc, S, sr, sc, g, (int)fast, W, stream);
  return PyLong_FromLong(rc);
}

/* gemm_strip_major(X, xr, xc, Wt, St, K, N, g, sw, version, Y, ws, ws_bytes, stream) */
static PyObject* py_sm_gemm(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 14, "gemm_strip_major")) return NULL;
  void *X, *Wt, *St, *Y, *ws, *stream;
  long long xr, xc, K, N, g, sw, ver, wsb;
  if (!take_ptr(a[0], &X) || !take_i64(a[1], &xr) || !take_i64(a[2], &xc) ||
      !take_ptr(a[3], &Wt) || !take_ptr(a[4], &St) || !take_i64(a[5], &K) ||
      !take_i64(a[6], &N) || !take_i64(a[7], &g) || !take_i64(a[8], &sw) ||
      !take_i64(a[9], &ver) || !take_ptr(a[10], &Y) || !take_ptr(a[11], &ws) ||
      !take_i64(a[12], &wsb) || !take_ptr(a[13], &stream))
    return NULL;
  return PyLong_FromLong(nibble_gemm_w4a16_strip_major(X, xr, xc, Wt, St, K, N, g, sw, ver, Y, ws,
                                                       (size_t)(wsb < 0 ? 0 : wsb), stream));
}

/* dequant_strip_major(Wt, St, K, N, g, sw, fast, W, stream) */
static PyObject* py_sm_dequant(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 9, "dequant_strip_major")) return NULL;
  void *Wt, *St, *W, *stream;
  long long K, N, g, sw, fast;
  if (!take_ptr(a[0], &Wt) || !take_ptr(a[1], &St) || !take_i64(a[2], &K) ||
      !take_i64(a[3], &N) || !take_i64(a[4], &g) || !take_i64(a[5], &sw) ||
      !take_i64(a[6], &fast) || !take_ptr(a[7], &W) || !take_ptr(a[8], &stream))
    return NULL;
  return PyLong_FromLong(nibble_dequant_w4_strip_major(Wt, St, K, N, g, sw, (int)fast, W, stream));
}

/* chain_create(stages: bytes of n packed nibble_chain_stage, n, M, stream) -> (status, handle) */
static PyObject* py_chain_create(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 4, "chain_create")) return NULL;
  long long count, M;
  void* stream;
  if (!PyBytes_Check(a[0])) {
    PyErr_SetString(PyExc_TypeError, "chain_create: stages must be bytes");
    return NULL;
  }
  if (!take_i64(a[1], &count) || !take_i64(a[2], &M) || !take_ptr(a[3], &stream)) return NULL;
  if (count < 0 || (size_t)PyBytes_GET_SIZE(a[0]) != (size_t)count * sizeof(nibble_chain_stage)) {
    PyErr_Format(PyExc_ValueError, "chain_create: %lld stages need %zu bytes, got %zd", count,
                 (size_t)count * sizeof(nibble_chain_stage), PyBytes_GET_SIZE(a[0]));
    return NULL;
  }
  void* chain = NULL;
  int rc = nibble_chain_create((const nibble_chain_stage*)PyBytes_AS_STRING(a[0]), count, M,
                               stream, &chain);
  PyObject* handle = NULL;
  if (rc == 0) {
    handle = PyLong_FromVoidPtr(chain);
    if (handle == NULL) {
      nibble_chain_destroy(chain);
      return NULL;
    }
  } else {
    Py_INCREF(Py_None);
    handle = Py_None;
  }
  return Py_BuildValue("(iN)", rc, handle);
}

/* chain_run(handle, timestamps, stream) */
static PyObject* py_chain_run(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 3, "chain_run")) return NULL;
  void *chain, *stamps, *stream;
  if (!take_ptr(a[0], &chain) || !take_ptr(a[1], &stamps) || !take_ptr(a[2], &stream)) return NULL;
  return PyLong_FromLong(nibble_chain_run(chain, stamps, stream));
}

/* chain_check(handle, stream) */
static PyObject* py_chain_check(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 2, "chain_check")) return NULL;
  void *chain, *stream;
  if (!take_ptr(a[0], &chain) || !take_ptr(a[1], &stream)) return NULL;
  return PyLong_FromLong(nibble_chain_check(chain, stream));
}

/* chain_info(handle, what) */
static PyObject* py_chain_info(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 2, "chain_info")) return NULL;
  void* chain;
  long long what;
  if (!take_ptr(a[0], &chain) || !take_i64(a[1], &what)) return NULL;
  return PyLong_FromLongLong(nibble_chain_info(chain, what));
}

/* chain_destroy(handle) */
static PyObject* py_chain_destroy(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  if (!nargs_is(n, 1, "chain_destroy")) return NULL;
  void* chain;
  if (!take_ptr(a[0], &chain)) return NULL;
  return PyLong_FromLong(nibble_chain_destroy(chain));
}

static PyObject* py_last_error(PyObject* self, PyObject* unused) {
  (void)self;
  (void)unused;
  return PyUnicode_FromString(nibble_last_error());
}

static PyObject* py_abi_version(PyObject* self, PyObject* unused) {
  (void)self;
  (void)unused;
  return PyLong_FromLong(nibble_abi_version());
}

static PyMethodDef kMethods[] = {
    {"gemv", (PyCFunction)(void (*)(void))py_gemv, METH_FASTCALL, "nibble_gemv_w4a16"},
    {"gemv_workspace_bytes", (PyCFunction)(void (*)(void))py_gemv_ws, METH_FASTCALL,
     "(nibble_gemv_workspace_bytes, nibble_gemv_counter_bytes)"},
    {"gemm", (PyCFunction)(void (*)(void))py_gemm, METH_FASTCALL, "nibble_gemm_w4a16"},
    {"gemm_workspace_bytes", (PyCFunction)(void (*)(void))py_gemm_ws, METH_FASTCALL,
     "(nibble_gemm_workspace_bytes, nibble_gemm_counter_bytes)"},
    {"dequant", (PyCFunction)(void (*)(void))py_dequant, METH_FASTCALL, "nibble_dequant_w4"},
    {"matmul_fused", (PyCFunction)(void (*)(void))py_fused, METH_FASTCALL,
     "nibble_matmul_w4a16_fused"},
    {"matmul_fused_workspace_bytes", (PyCFunction)(void (*)(void))py_fused_ws, METH_FASTCALL,
     "nibble_matmul_fused_workspace_bytes / nibble_matmul_fused_counter_bytes"},
    {"gemm_streams", (PyCFunction)(void (*)(void))py_gemm_streams, METH_FASTCALL,
     "nibble_gemm_streams"},
    {"strip_major_cols", (PyCFunction)(void (*)(void))py_sm_cols, METH_FASTCALL,
     "nibble_strip_major_cols"},
    {"gemv_timeline", (PyCFunction)(void (*)(void))py_gemv_timeline, METH_FASTCALL,
     "nibble_gemv_timeline"},
    {"chain_strip_cols", (PyCFunction)(void (*)(void))py_chain_cols, METH_FASTCALL,
     "nibble_chain_strip_cols"},
    {"pack_strip_major", (PyCFunction)(void (*)(void))py_sm_pack, METH_FASTCALL,
     "nibble_pack_strip_major"},
    {"gemv_strip_major", (PyCFunction)(void (*)(void))py_sm_gemv, METH_FASTCALL,
     "nibble_gemv_w4a16_strip_major"},
    {"gemm_strip_major", (PyCFunction)(void (*)(void))py_sm_gemm, METH_FASTCALL,
     "nibble_gemm_w4a16_strip_major"},
    {"dequant_strip_major", (PyCFunction)(void (*)(void))py_sm_dequant, METH_FASTCALL,
     "nibble_dequant_w4_strip_major"},
    {"rmsnorm", (PyCFunction)(void (*)(void))py_rmsnorm, METH_FASTCALL, "nibble_rmsnorm_f16"},
    {"attention", (PyCFunction)(void (*)(void))py_attention, METH_FASTCALL,
     "nibble_attention_decode_f16"},
    {"attention_workspace_bytes", (PyCFunction)(void (*)(void))py_attention_ws, METH_FASTCALL,
     "(nibble_attention_decode_workspace_bytes, nibble_attention_decode_counter_bytes)"},
    {"chain_create", (PyCFunction)(void (*)(void))py_chain_create, METH_FASTCALL,
     "nibble_chain_create"},
    {"chain_run", (PyCFunction)(void (*)(void))py_chain_run, METH_FASTCALL, "nibble_chain_run"},
    {"chain_check", (PyCFunction)(void (*)(void))py_chain_check, METH_FASTCALL,
     "nibble_chain_check"},
    {"chain_info", (PyCFunction)(void (*)(void))py_chain_info, METH_FASTCALL, "nibble_chain_info"},
    {"chain_destroy", (PyCFunction)(void (*)(void))py_chain_destroy, METH_FASTCALL,
     "nibble_chain_destroy"},
    {"last_error", py_last_error, METH_NOARGS, "nibble_last_error"},
    {"abi_version", py_abi_version, METH_NOARGS, "nibble_abi_version"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_binding",
                                     "CPython binding over the nibblegemm_amd C ABI", -1, kMethods,
                                     NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__binding(void) { return PyModule_Create(&kModule); }
