// Node.js N-API addon over the ns2 C ABI (include/ns2.h).
//
// Device buffers cross into JavaScript as BigInt addresses; sizes, strides and offsets as
// Numbers; null/undefined stands for a NULL pointer. Every wrapper calls exactly one C entry
// point and turns a non-zero status into a thrown JS Error carrying ns2_last_error(), the
// way the reference's WebGPU runtime surfaces validation and device-loss errors
// (app/gpu/device.js:97-102, 171, 224-231).
#include <node_api.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "ns2.h"

namespace {

struct Ctx {
  napi_env env;
  napi_value* argv;
  size_t argc;
  bool failed = false;

  void fail(const std::string& msg) {
    if (!failed) napi_throw_error(env, nullptr, msg.c_str());
    failed = true;
  }
  napi_valuetype type(size_t i) {
    napi_valuetype t = napi_undefined;
    if (i < argc) napi_typeof(env, argv[i], &t);
    return t;
  }
  void* ptr(size_t i) {
    napi_valuetype t = type(i);
    if (t == napi_null || t == napi_undefined) return nullptr;
    if (t != napi_bigint) {
      fail("argument " + std::to_string(i) + ": expected a BigInt device address or null");
      return nullptr;
    }
    uint64_t v = 0;
    bool lossless = true;
    napi_get_value_bigint_uint64(env, argv[i], &v, &lossless);
    return reinterpret_cast<void*>(static_cast<uintptr_t>(v));
  }
  int64_t i64(size_t i) {
    napi_valuetype t = type(i);
    if (t == napi_bigint) {
      int64_t v = 0;
      bool lossless = true;
      napi_get_value_bigint_int64(env, argv[i], &v, &lossless);
      return v;
    }
    if (t != napi_number) {
      fail("argument " + std::to_string(i) + ": expected a number");
      return 0;
    }
    int64_t v = 0;
    napi_get_value_int64(env, argv[i], &v);
    return v;
  }
  int i32(size_t i) { return static_cast<int>(i64(i)); }
  double f64(size_t i) {
    if (type(i) != napi_number) {
      fail("argument " + std::to_string(i) + ": expected a number");
      return 0;
    }
    double v = 0;
    napi_get_value_double(env, argv[i], &v);
    return v;
  }
  float f32(size_t i) { return static_cast<float>(f64(i)); }
};

template <size_t N>
bool get_args(napi_env env, napi_callback_info info, napi_value (&argv)[N], size_t* argc) {
  *argc = N;
  return napi_get_cb_info(env, info, argc, argv, nullptr, nullptr) == napi_ok;
}

napi_value undef(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

napi_value check(napi_env env, Ctx& c, int rc) {
  if (c.failed) return nullptr;
  if (rc != NS2_OK) {
    napi_throw_error(env, nullptr, ns2_last_error());
    return nullptr;
  }
  return undef(env);
}

napi_value bigint(napi_env env, void* p) {
  napi_value v;
  napi_create_bigint_uint64(env, reinterpret_cast<uintptr_t>(p), &v);
  return v;
}

napi_value number(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

#define ARGS(n)              \
  napi_value argv[n];        \
  size_t argc;               \
  get_args(env, info, argv, &argc); \
  Ctx c{env, argv, argc};

// ---- runtime ------------------------------------------------------------------------------

napi_value Init(napi_env env, napi_callback_info info) {
  ARGS(1);
  int dev = c.type(0) == napi_number ? c.i32(0) : 0;
  return check(env, c, ns2_init(dev));
}

napi_value DeviceInfo(napi_env env, napi_callback_info info) {
  char name[256];
  int cus = 0;
  size_t hbm = 0;
  if (ns2_device_info(name, sizeof(name), &cus, &hbm) != NS2_OK) {
    napi_throw_error(env, nullptr, ns2_last_error());
    return nullptr;
  }
  napi_value o, s;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &s);
  napi_set_named_property(env, o, "name", s);
  napi_set_named_property(env, o, "computeUnits", number(env, cus));
  napi_set_named_property(env, o, "hbmBytes", number(env, (double)hbm));
  return o;
}

napi_value Malloc(napi_env env, napi_callback_info info) {
  ARGS(1);
  size_t bytes = (size_t)c.i64(0);
  void* p = nullptr;
  if (!check(env, c, c.failed ? 0 : ns2_malloc(&p, bytes))) return nullptr;
  return bigint(env, p);
}

napi_value Free(napi_env env, napi_callback_info info) {
  ARGS(1);
  void* p = c.ptr(0);
  return check(env, c, c.failed ? 0 : ns2_free(p));
}

napi_value PoolRound(napi_env env, napi_callback_info info) {
  ARGS(1);
  size_t b = (size_t)c.i64(0);
  if (c.failed) return nullptr;
  return number(env, (double)ns2_pool_round(b));
}

napi_value PoolGet(napi_env env, napi_callback_info info) {
  ARGS(1);
  size_t bytes = (size_t)c.i64(0);
  void* p = nullptr;
  size_t rounded = 0;
  if (!check(env, c, c.failed ? 0 : ns2_pool_get(bytes, &p, &rounded))) return nullptr;
  napi_value arr;
  napi_create_array_with_length(env, 2, &arr);
  napi_set_element(env, arr, 0, bigint(env, p));
  napi_set_element(env, arr, 1, number(env, (double)rounded));
  return arr;
}

napi_value PoolPut(napi_env env, napi_callback_info info) {
  ARGS(2);
  void* p = c.ptr(0);
  size_t r = (size_t)c.i64(1);
  return check(env, c, c.failed ? 0 : ns2_pool_put(p, r));
}

napi_value PoolTrim(napi_env env, napi_callback_info info) {
  Ctx c{env, nullptr, 0};
  return check(env, c, ns2_pool_trim());
}

napi_value PoolStats(napi_env env, napi_callback_info info) {
  size_t a = 0, p = 0;
  ns2_pool_stats(&a, &p);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "allocated", number(env, (double)a));
  napi_set_named_property(env, o, "peak", number(env, (double)p));
  return o;
}

// h2d(dst, typedArrayOrBuffer[, dstByteOffset])
napi_value H2D(napi_env env, napi_callback_info info) {
  ARGS(3);
  char* dst = static_cast<char*>(c.ptr(0));
  int64_t off = c.type(2) == napi_number ? c.i64(2) : 0;
  if (c.failed) return nullptr;
  void* data = nullptr;
  size_t bytes = 0;
  bool is_ta = false, is_ab = false, is_dv = false;
  napi_is_typedarray(env, argv[1], &is_ta);
  napi_is_arraybuffer(env, argv[1], &is_ab);
  napi_is_dataview(env, argv[1], &is_dv);
  if (is_ta) {
    napi_typedarray_type t;
    size_t len, boff;
    napi_value ab;
    napi_get_typedarray_info(env, argv[1], &t, &len, &data, &ab, &boff);
    size_t es = 1;
    switch (t) {
      case napi_int16_array: case napi_uint16_array: es = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
      default: es = 1;
    }
    bytes = len * es;
  } else if (is_ab) {
    napi_get_arraybuffer_info(env, argv[1], &data, &bytes);
  } else if (is_dv) {
    napi_value ab;
    size_t boff;
    napi_get_dataview_info(env, argv[1], &bytes, &data, &ab, &boff);
  } else {
    c.fail("h2d: expected a TypedArray, ArrayBuffer or DataView");
    return nullptr;
  }
  return check(env, c, ns2_h2d(dst + off, data, bytes));
}

// d2h(src, dstTypedArray) or d2h(src, bytes) -> ArrayBuffer
napi_value D2H(napi_env env, napi_callback_info info) {
  ARGS(2);
  const void* src = c.ptr(0);
  if (c.failed) return nullptr;
  bool is_ta = false;
  napi_is_typedarray(env, argv[1], &is_ta);
  if (is_ta) {
    napi_typedarray_type t;
    size_t len, boff;
    void* data;
    napi_value ab;
    napi_get_typedarray_info(env, argv[1], &t, &len, &data, &ab, &boff);
    size_t es = (t == napi_float32_array || t == napi_int32_array || t == napi_uint32_array) ? 4
                : (t == napi_int16_array || t == napi_uint16_array) ? 2
                : (t == napi_float64_array) ? 8 : 1;
    if (!check(env, c, ns2_d2h(data, src, len * es))) return nullptr;
    return argv[1];
  }
  size_t bytes = (size_t)c.i64(1);
  if (c.failed) return nullptr;
  void* data = nullptr;
  napi_value ab;
  napi_create_arraybuffer(env, bytes, &data, &ab);
  if (!check(env, c, ns2_d2h(data, src, bytes))) return nullptr;
  return ab;
}

napi_value Sync(napi_env env, napi_callback_info info) {
  Ctx c{env, nullptr, 0};
  return check(env, c, ns2_sync());
}

napi_value Fill(napi_env env, napi_callback_info info) {
  ARGS(3);
  void* p = c.ptr(0);
  uint32_t v = (uint32_t)c.i64(1);
  size_t n = (size_t)c.i64(2);
  return check(env, c, c.failed ? 0 : ns2_fill_u32(p, v, n));
}

// graphBegin() / graphEnd() -> BigInt handle / graphLaunch(h) / graphDestroy(h)
napi_value GraphBegin(napi_env env, napi_callback_info info) {
  Ctx c{env, nullptr, 0};
  return check(env, c, ns2_graph_begin());
}

napi_value GraphEnd(napi_env env, napi_callback_info info) {
  void* g = nullptr;
  if (ns2_graph_end(&g) != NS2_OK) {
    napi_throw_error(env, nullptr, ns2_last_error());
    return nullptr;
  }
  return bigint(env, g);
}

napi_value GraphLaunch(napi_env env, napi_callback_info info) {
  ARGS(1);
  void* g = c.ptr(0);
  return check(env, c, c.failed ? 0 : ns2_graph_launch(g));
}

napi_value GraphDestroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  void* g = c.ptr(0);
  return check(env, c, c.failed ? 0 : ns2_graph_destroy(g));
}

napi_value EventCreate(napi_env env, napi_callback_info info) {
  void* ev = nullptr;
  if (ns2_event_create(&ev) != NS2_OK) {
    napi_throw_error(env, nullptr, ns2_last_error());
    return nullptr;
  }
  return bigint(env, ev);
}

napi_value EventRecord(napi_env env, napi_callback_info info) {
  ARGS(1);
  void* ev = c.ptr(0);
  return check(env, c, c.failed ? 0 : ns2_event_record(ev));
}

napi_value EventElapsed(napi_env env, napi_callback_info info) {
  ARGS(2);
  void* a = c.ptr(0);
  void* b = c.ptr(1);
  float ms = 0;
  if (!check(env, c, c.failed ? 0 : ns2_event_elapsed(a, b, &ms))) return nullptr;
  return number(env, ms);
}

napi_value EventDestroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  void* ev = c.ptr(0);
  return check(env, c, c.failed ? 0 : ns2_event_destroy(ev));
}

napi_value ProfileEnable(napi_env env, napi_callback_info info) {
  ARGS(1);
  int on = c.i32(0);
  return check(env, c, c.failed ? 0 : ns2_profile_enable(on));
}

napi_value ProfileReset(napi_env env, napi_callback_info info) {
  Ctx c{env, nullptr, 0};
  return check(env, c, ns2_profile_reset());
}

// profileReport() -> JSON text {"kernel": {"count", "ms"}}
napi_value ProfileReport(napi_env env, napi_callback_info info) {
  std::string buf(1 << 16, '\0');
  if (ns2_profile_report(&buf[0], buf.size()) != NS2_OK) {
    napi_throw_error(env, nullptr, ns2_last_error());
    return nullptr;
  }
  napi_value s;
  napi_create_string_utf8(env, buf.c_str(), NAPI_AUTO_LENGTH, &s);
  return s;
}

// ---- ops ------------------------------------------------------------------------------------

napi_value Hadamard256(napi_env env, napi_callback_info info) {
  ARGS(3);
  auto x = (const float*)c.ptr(0);
  auto y = (float*)c.ptr(1);
  long long g = c.i64(2);
  return check(env, c, c.failed ? 0 : ns2_hadamard256(x, y, g));
}

// rotateF16(x, ldx, y, ldy, rows, cols, tiled)
napi_value RotateF16(napi_env env, napi_callback_info info) {
  ARGS(7);
  auto x = (const float*)c.ptr(0);
  int ldx = c.i32(1);
  auto y = (uint16_t*)c.ptr(2);
  int ldy = c.i32(3), rows = c.i32(4), cols = c.i32(5), tiled = c.i32(6);
  return check(env, c, c.failed ? 0 : ns2_rotate_f16(x, ldx, y, ldy, rows, cols, tiled));
}

// tileI8Weight(W, Wt, N, K)
napi_value TileI8Weight(napi_env env, napi_callback_info info) {
  ARGS(4);
  auto W = (const int8_t*)c.ptr(0);
  auto Wt = (int8_t*)c.ptr(1);
  int N = c.i32(2), K = c.i32(3);
  return check(env, c, c.failed ? 0 : ns2_tile_i8_weight(W, Wt, N, K));
}

// tileI8WeightGlu(W, Wt, N, K)
napi_value TileI8WeightGlu(napi_env env, napi_callback_info info) {
  ARGS(4);
  auto W = (const int8_t*)c.ptr(0);
  auto Wt = (int8_t*)c.ptr(1);
  int N = c.i32(2), K = c.i32(3);
  return check(env, c, c.failed ? 0 : ns2_tile_i8_weight_glu(W, Wt, N, K));
}

// linearI8GluRotTiled(At, Wt, scale, bias, Y, M, N, K, alpha, act[, loraA, loraB, loraR])
napi_value LinearI8GluRotTiled(napi_env env, napi_callback_info info) {
  ARGS(13);
  auto At = (const uint16_t*)c.ptr(0);
  auto Wt = (const int8_t*)c.ptr(1);
  auto scale = (const float*)c.ptr(2);
  auto bias = (const float*)c.ptr(3);
  auto Y = (uint16_t*)c.ptr(4);
  int M = c.i32(5), N = c.i32(6), K = c.i32(7);
  float alpha = c.f32(8);
  int act = c.i32(9);
  // optional LoRA side path: loraA, loraB (device addresses), loraR (0: none)
  auto la = (const uint16_t*)c.ptr(10);
  auto lb = (const uint16_t*)c.ptr(11);
  int lr = c.type(12) == napi_number ? c.i32(12) : 0;
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_i8_glu_rot_tiled_lora(At, Wt, scale, bias, Y, M, N, K, alpha, act, la, lb, lr));
}

// linearI8Tiled(At, Wt, scale, bias, C, M, N, K, ldc, cOff, alpha, act, resid, gate, gOff[, loraA, loraB, loraR])
napi_value LinearI8Tiled(napi_env env, napi_callback_info info) {
  ARGS(18);
  auto At = (const uint16_t*)c.ptr(0);
  auto Wt = (const int8_t*)c.ptr(1);
  auto scale = (const float*)c.ptr(2);
  auto bias = (const float*)c.ptr(3);
  auto C = (float*)c.ptr(4);
  int M = c.i32(5), N = c.i32(6), K = c.i32(7), ldc = c.i32(8);
  long long cOff = c.i64(9);
  float alpha = c.f32(10);
  int act = c.i32(11), resid = c.i32(12);
  auto gate = (const float*)c.ptr(13);
  long long gOff = c.i64(14);
  // optional LoRA side path: loraA, loraB (device addresses), loraR (0: none)
  auto la = (const uint16_t*)c.ptr(15);
  auto lb = (const uint16_t*)c.ptr(16);
  int lr = c.type(17) == napi_number ? c.i32(17) : 0;
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_i8_tiled_lora(At, Wt, scale, bias, C, M, N, K, ldc, cOff, alpha, act, resid, gate, gOff, la, lb, lr));
}

// tileBf16Weight(W, Wt, N, K)
napi_value TileBf16Weight(napi_env env, napi_callback_info info) {
  ARGS(4);
  auto W = (const uint16_t*)c.ptr(0);
  auto Wt = (uint16_t*)c.ptr(1);
  int N = c.i32(2), K = c.i32(3);
  return check(env, c, c.failed ? 0 : ns2_tile_bf16_weight(W, Wt, N, K));
}

// linearF16wTiled(At, Wt, bias, C, M, N, K, ldc, cOff, alpha, act, resid, gate, gOff[, loraA, loraB, loraR])
napi_value LinearF16wTiled(napi_env env, napi_callback_info info) {
  ARGS(17);
  auto At = (const uint16_t*)c.ptr(0);
  auto Wt = (const uint16_t*)c.ptr(1);
  auto bias = (const float*)c.ptr(2);
  auto C = (float*)c.ptr(3);
  int M = c.i32(4), N = c.i32(5), K = c.i32(6), ldc = c.i32(7);
  long long cOff = c.i64(8);
  float alpha = c.f32(9);
  int act = c.i32(10), resid = c.i32(11);
  auto gate = (const float*)c.ptr(12);
  long long gOff = c.i64(13);
  auto la = (const uint16_t*)c.ptr(14);
  auto lb = (const uint16_t*)c.ptr(15);
  int lr = c.type(16) == napi_number ? c.i32(16) : 0;
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_f16w_tiled_lora(At, Wt, bias, C, M, N, K, ldc, cOff, alpha, act, resid, gate, gOff,
                                                  la, lb, lr));
}

// toTiledF16(x, ldx, sub, ldsub, y, rows, cols)
napi_value ToTiledF16(napi_env env, napi_callback_info info) {
  ARGS(7);
  auto x = (const float*)c.ptr(0);
  int ldx = c.i32(1);
  auto sub = (const float*)c.ptr(2);
  int ldsub = c.i32(3);
  auto y = (uint16_t*)c.ptr(4);
  int rows = c.i32(5), cols = c.i32(6);
  return check(env, c, c.failed ? 0 : ns2_to_tiled_f16(x, ldx, sub, ldsub, y, rows, cols));
}

// linearI8(A, aFmt, lda, W, scale, bias, add, C, M, N, K, ldc, cOff, alpha, act, resid, gate, gOff[, loraA, loraB, loraR])
napi_value LinearI8(napi_env env, napi_callback_info info) {
  ARGS(21);
  const void* A = c.ptr(0);
  int aFmt = c.i32(1), lda = c.i32(2);
  auto W = (const int8_t*)c.ptr(3);
  auto scale = (const float*)c.ptr(4);
  auto bias = (const float*)c.ptr(5);
  auto add = (const float*)c.ptr(6);
  auto C = (float*)c.ptr(7);
  int M = c.i32(8), N = c.i32(9), K = c.i32(10), ldc = c.i32(11);
  long long cOff = c.i64(12);
  float alpha = c.f32(13);
  int act = c.i32(14), resid = c.i32(15);
  auto gate = (const float*)c.ptr(16);
  long long gOff = c.i64(17);
  // optional LoRA side path: loraA, loraB (device addresses), loraR (0: none)
  auto la = (const uint16_t*)c.ptr(18);
  auto lb = (const uint16_t*)c.ptr(19);
  int lr = c.type(20) == napi_number ? c.i32(20) : 0;
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_i8_lora(A, aFmt, lda, W, scale, bias, add, C, M, N, K, ldc, cOff, alpha, act, resid, gate, gOff, la, lb, lr));
}

// linearBf16(A, lda, W, bias, add, C, M, N, K, ldc, cOff, alpha, act, resid, gate, gOff[, loraA, loraB, loraR])
napi_value LinearBf16(napi_env env, napi_callback_info info) {
  ARGS(19);
  auto A = (const float*)c.ptr(0);
  int lda = c.i32(1);
  auto W = (const uint16_t*)c.ptr(2);
  auto bias = (const float*)c.ptr(3);
  auto add = (const float*)c.ptr(4);
  auto C = (float*)c.ptr(5);
  int M = c.i32(6), N = c.i32(7), K = c.i32(8), ldc = c.i32(9);
  long long cOff = c.i64(10);
  float alpha = c.f32(11);
  int act = c.i32(12), resid = c.i32(13);
  auto gate = (const float*)c.ptr(14);
  long long gOff = c.i64(15);
  // optional LoRA side path: loraA, loraB (device addresses), loraR (0: none)
  auto la = (const uint16_t*)c.ptr(16);
  auto lb = (const uint16_t*)c.ptr(17);
  int lr = c.type(18) == napi_number ? c.i32(18) : 0;
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_bf16_lora(A, lda, W, bias, add, C, M, N, K, ldc, cOff, alpha, act, resid, gate, gOff, la, lb, lr));
}

// attention(q, k, v, o, batch, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, oOff,
//           qBatch, kBatch, vBatch, oBatch, scale, keyBias, biasStart, biasBatch,
//           qNorm, kNorm, eps, ropeCs, sinOff, ropeRows)
napi_value Attention(napi_env env, napi_callback_info info) {
  ARGS(31);
  auto q = (const float*)c.ptr(0);
  auto k = (const float*)c.ptr(1);
  auto v = (const float*)c.ptr(2);
  auto o = (float*)c.ptr(3);
  int batch = c.i32(4), Lq = c.i32(5), Lk = c.i32(6), H = c.i32(7), D = c.i32(8);
  int ldq = c.i32(9), ldk = c.i32(10), ldv = c.i32(11), ldo = c.i32(12);
  long long qOff = c.i64(13), kOff = c.i64(14), vOff = c.i64(15), oOff = c.i64(16);
  long long qB = c.i64(17), kB = c.i64(18), vB = c.i64(19), oB = c.i64(20);
  float scale = c.f32(21);
  auto kb = (const float*)c.ptr(22);
  int biasStart = c.i32(23);
  long long biasBatch = c.i64(24);
  auto qn = (const float*)c.ptr(25);
  auto kn = (const float*)c.ptr(26);
  float eps = c.f32(27);
  auto cs = (const float*)c.ptr(28);
  long long sinOff = c.i64(29);
  int ropeRows = c.i32(30);
  if (c.failed) return nullptr;
  return check(env, c, ns2_attention(q, k, v, o, batch, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, oOff,
                                     qB, kB, vB, oB, scale, kb, biasStart, biasBatch, qn, kn, eps, cs, sinOff, ropeRows));
}

// linearI8TiledVpack(At, Wt, scale, bias, C, M, N, K, ldc, cOff, alpha, act, loraA, loraB, loraR, vpk, vcol0,
//                    H, D, Lk)
napi_value LinearI8TiledVpack(napi_env env, napi_callback_info info) {
  ARGS(20);
  auto At = (const uint16_t*)c.ptr(0);
  auto Wt = (const int8_t*)c.ptr(1);
  auto scale = (const float*)c.ptr(2);
  auto bias = (const float*)c.ptr(3);
  auto C = (float*)c.ptr(4);
  int M = c.i32(5), N = c.i32(6), K = c.i32(7), ldc = c.i32(8);
  long long cOff = c.i64(9);
  float alpha = c.f32(10);
  int act = c.i32(11);
  auto la = (const uint16_t*)c.ptr(12);
  auto lb = (const uint16_t*)c.ptr(13);
  int lr = c.type(14) == napi_number ? c.i32(14) : 0;
  auto vpk = (uint16_t*)c.ptr(15);
  int vcol0 = c.i32(16), H = c.i32(17), D = c.i32(18), Lk = c.i32(19);
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_i8_tiled_vpack(At, Wt, scale, bias, C, M, N, K, ldc, cOff, alpha, act, la, lb, lr,
                                                 vpk, vcol0, H, D, Lk));
}

// attentionVpackBytes(Lk, H, D) -> bytes of a packed-value buffer
napi_value AttentionVpackBytes(napi_env env, napi_callback_info info) {
  ARGS(3);
  int Lk = c.i32(0), H = c.i32(1), D = c.i32(2);
  if (c.failed) return nullptr;
  napi_value r;
  napi_create_double(env, (double)ns2_attention_vpack_bytes(Lk, H, D), &r);
  return r;
}

// attentionVpacked(q, k, v, o, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, oOff, scale, keyBias,
//                  biasStart, qNorm, kNorm, eps, ropeCs, sinOff, ropeRows, kText, vText, ldText, textStart,
//                  vpk, vRows)
napi_value AttentionVpacked(napi_env env, napi_callback_info info) {
  ARGS(31);
  auto q = (const float*)c.ptr(0);
  auto k = (const float*)c.ptr(1);
  auto v = (const float*)c.ptr(2);
  auto o = (float*)c.ptr(3);
  int Lq = c.i32(4), Lk = c.i32(5), H = c.i32(6), D = c.i32(7);
  int ldq = c.i32(8), ldk = c.i32(9), ldv = c.i32(10), ldo = c.i32(11);
  long long qOff = c.i64(12), kOff = c.i64(13), vOff = c.i64(14), oOff = c.i64(15);
  float scale = c.f32(16);
  auto kb = (const float*)c.ptr(17);
  int biasStart = c.i32(18);
  auto qn = (const float*)c.ptr(19);
  auto kn = (const float*)c.ptr(20);
  float eps = c.f32(21);
  auto cs = (const float*)c.ptr(22);
  long long sinOff = c.i64(23);
  int ropeRows = c.i32(24);
  auto kt = (const float*)c.ptr(25);
  auto vt = (const float*)c.ptr(26);
  int ldText = c.i32(27), textStart = c.i32(28);
  auto vpk = (uint16_t*)c.ptr(29);
  int vRows = c.i32(30);
  if (c.failed) return nullptr;
  return check(env, c, ns2_attention_vpacked(q, k, v, o, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, oOff,
                                             scale, kb, biasStart, qn, kn, eps, cs, sinOff, ropeRows, kt, vt, ldText,
                                             textStart, vpk, vRows));
}

// attentionText(q, k, v, o, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, oOff, scale, keyBias,
//               biasStart, qNorm, kNorm, eps, ropeCs, sinOff, ropeRows, kText, vText, ldText, textStart)
napi_value AttentionText(napi_env env, napi_callback_info info) {
  ARGS(29);
  auto q = (const float*)c.ptr(0);
  auto k = (const float*)c.ptr(1);
  auto v = (const float*)c.ptr(2);
  auto o = (float*)c.ptr(3);
  int Lq = c.i32(4), Lk = c.i32(5), H = c.i32(6), D = c.i32(7);
  int ldq = c.i32(8), ldk = c.i32(9), ldv = c.i32(10), ldo = c.i32(11);
  long long qOff = c.i64(12), kOff = c.i64(13), vOff = c.i64(14), oOff = c.i64(15);
  float scale = c.f32(16);
  auto kb = (const float*)c.ptr(17);
  int biasStart = c.i32(18);
  auto qn = (const float*)c.ptr(19);
  auto kn = (const float*)c.ptr(20);
  float eps = c.f32(21);
  auto cs = (const float*)c.ptr(22);
  long long sinOff = c.i64(23);
  int ropeRows = c.i32(24);
  auto kt = (const float*)c.ptr(25);
  auto vt = (const float*)c.ptr(26);
  int ldText = c.i32(27), textStart = c.i32(28);
  if (c.failed) return nullptr;
  return check(env, c, ns2_attention_text(q, k, v, o, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, oOff, scale,
                                          kb, biasStart, qn, kn, eps, cs, sinOff, ropeRows, kt, vt, ldText, textStart));
}

// attentionRows(q, k, v, o, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, group, causal)
napi_value AttentionRows(napi_env env, napi_callback_info info) {
  ARGS(17);
  auto q = (const float*)c.ptr(0);
  auto k = (const float*)c.ptr(1);
  auto v = (const float*)c.ptr(2);
  auto o = (float*)c.ptr(3);
  int Lq = c.i32(4), Lk = c.i32(5), H = c.i32(6), D = c.i32(7);
  int ldq = c.i32(8), ldk = c.i32(9), ldv = c.i32(10), ldo = c.i32(11);
  long long qOff = c.i64(12), kOff = c.i64(13), vOff = c.i64(14);
  int group = c.i32(15), causal = c.i32(16);
  if (c.failed) return nullptr;
  return check(env, c, ns2_attention_rows(q, k, v, o, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, group, causal));
}

// attentionRowsF16kv(q, k, v, o, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, group, causal):
// k and v fp16, their strides and offsets in fp16 elements
napi_value AttentionRowsF16kv(napi_env env, napi_callback_info info) {
  ARGS(17);
  auto q = (const float*)c.ptr(0);
  auto k = (const uint16_t*)c.ptr(1);
  auto v = (const uint16_t*)c.ptr(2);
  auto o = (float*)c.ptr(3);
  int Lq = c.i32(4), Lk = c.i32(5), H = c.i32(6), D = c.i32(7);
  int ldq = c.i32(8), ldk = c.i32(9), ldv = c.i32(10), ldo = c.i32(11);
  long long qOff = c.i64(12), kOff = c.i64(13), vOff = c.i64(14);
  int group = c.i32(15), causal = c.i32(16);
  if (c.failed) return nullptr;
  return check(env, c,
               ns2_attention_rows_f16kv(q, k, v, o, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff, vOff, group, causal));
}

// attentionRowsF16kvOproj(q, k, v, woTiled, part, Lq, Lk, H, D, ldq, ldk, ldv, qOff, kOff, vOff, group, causal, N)
napi_value AttentionRowsF16kvOproj(napi_env env, napi_callback_info info) {
  ARGS(18);
  auto q = (const float*)c.ptr(0);
  auto k = (const uint16_t*)c.ptr(1);
  auto v = (const uint16_t*)c.ptr(2);
  auto wo = (const uint16_t*)c.ptr(3);
  auto part = (float*)c.ptr(4);
  int Lq = c.i32(5), Lk = c.i32(6), H = c.i32(7), D = c.i32(8);
  int ldq = c.i32(9), ldk = c.i32(10), ldv = c.i32(11);
  long long qOff = c.i64(12), kOff = c.i64(13), vOff = c.i64(14);
  int group = c.i32(15), causal = c.i32(16), N = c.i32(17);
  if (c.failed) return nullptr;
  return check(env, c, ns2_attention_rows_f16kv_oproj(q, k, v, wo, part, Lq, Lk, H, D, ldq, ldk, ldv, qOff, kOff, vOff,
                                                      group, causal, N));
}

// partsAddRmsnorm(part, splits, bias, x, wAdd, wOut, y, M, N, eps)
napi_value PartsAddRmsnorm(napi_env env, napi_callback_info info) {
  ARGS(10);
  auto part = (const float*)c.ptr(0);
  int splits = c.i32(1);
  auto bias = (const float*)c.ptr(2);
  auto x = (float*)c.ptr(3);
  auto wAdd = (const float*)c.ptr(4);
  auto wOut = (const float*)c.ptr(5);
  auto y = (float*)c.ptr(6);
  int M = c.i32(7), N = c.i32(8);
  float eps = c.f32(9);
  if (c.failed) return nullptr;
  return check(env, c, ns2_parts_add_rmsnorm(part, splits, bias, x, wAdd, wOut, y, M, N, eps));
}

// headNorm(X, w, L, H, D, ld, colOff, rowOff, cs, sinOff, eps)
napi_value HeadNorm(napi_env env, napi_callback_info info) {
  ARGS(11);
  auto X = (float*)c.ptr(0);
  auto w = (const float*)c.ptr(1);
  int L = c.i32(2), H = c.i32(3), D = c.i32(4), ld = c.i32(5);
  long long colOff = c.i64(6), rowOff = c.i64(7);
  auto cs = (const float*)c.ptr(8);
  long long sinOff = c.i64(9);
  float eps = c.f32(10);
  if (c.failed) return nullptr;
  return check(env, c, ns2_head_norm(X, w, L, H, D, ld, colOff, rowOff, cs, sinOff, eps));
}

// headNorm2(X, w1, H1, w2, H2, L, D, ld, colOff, rowOff, cs, sinOff, eps)
napi_value HeadNorm2(napi_env env, napi_callback_info info) {
  ARGS(13);
  auto X = (float*)c.ptr(0);
  auto w1 = (const float*)c.ptr(1);
  int H1 = c.i32(2);
  auto w2 = (const float*)c.ptr(3);
  int H2 = c.i32(4), L = c.i32(5), D = c.i32(6), ld = c.i32(7);
  long long colOff = c.i64(8), rowOff = c.i64(9);
  auto cs = (const float*)c.ptr(10);
  long long sinOff = c.i64(11);
  float eps = c.f32(12);
  if (c.failed) return nullptr;
  return check(env, c, ns2_head_norm2(X, w1, H1, w2, H2, L, D, ld, colOff, rowOff, cs, sinOff, eps));
}

// normMod(x, mod, shiftOff, scaleOff, rows, cols, weight, eps, y) /
// normModRotateF16(x, mod, shiftOff, scaleOff, rows, cols, weight, eps, y, tiled)
template <bool ROT>
napi_value NormModT(napi_env env, napi_callback_info info) {
  ARGS(10);
  auto x = (const float*)c.ptr(0);
  auto mod = (const float*)c.ptr(1);
  long long sh = c.i64(2), sc = c.i64(3);
  int rows = c.i32(4), cols = c.i32(5);
  auto w = (const float*)c.ptr(6);
  float eps = c.f32(7);
  void* y = c.ptr(8);
  int tiled = ROT ? c.i32(9) : 0;
  if (c.failed) return nullptr;
  int rc = ROT ? ns2_norm_mod_rotate_f16(x, mod, sh, sc, rows, cols, w, eps, (uint16_t*)y, tiled)
               : ns2_norm_mod(x, mod, sh, sc, rows, cols, w, eps, (float*)y);
  return check(env, c, rc);
}

// normModF16(x, mod, shiftOff, scaleOff, rows, cols, weight, eps, y, tiled)
napi_value NormModF16(napi_env env, napi_callback_info info) {
  ARGS(10);
  auto x = (const float*)c.ptr(0);
  auto mod = (const float*)c.ptr(1);
  long long sh = c.i64(2), sc = c.i64(3);
  int rows = c.i32(4), cols = c.i32(5);
  auto w = (const float*)c.ptr(6);
  float eps = c.f32(7);
  auto y = (uint16_t*)c.ptr(8);
  int tiled = c.i32(9);
  if (c.failed) return nullptr;
  return check(env, c, ns2_norm_mod_f16(x, mod, sh, sc, rows, cols, w, eps, y, tiled));
}

// glu(x, y, rows, I, act) / gluRotateF16(x, y, rows, I, act, tiled)
template <bool ROT>
napi_value GluT(napi_env env, napi_callback_info info) {
  ARGS(6);
  auto x = (const float*)c.ptr(0);
  void* y = c.ptr(1);
  int rows = c.i32(2), I = c.i32(3), act = c.i32(4);
  int tiled = ROT ? c.i32(5) : 0;
  if (c.failed) return nullptr;
  int rc = ROT ? ns2_glu_rotate_f16(x, (uint16_t*)y, rows, I, act, tiled) : ns2_glu(x, (float*)y, rows, I, act);
  return check(env, c, rc);
}

// elementwise(op, a, b, y, n)
napi_value Elementwise(napi_env env, napi_callback_info info) {
  ARGS(5);
  int op = c.i32(0);
  auto a = (const float*)c.ptr(1);
  auto b = (const float*)c.ptr(2);
  auto y = (float*)c.ptr(3);
  long long n = c.i64(4);
  if (c.failed) return nullptr;
  return check(env, c, ns2_elementwise(op, a, b, y, n));
}

napi_value Accumulate(napi_env env, napi_callback_info info) {
  ARGS(3);
  auto y = (float*)c.ptr(0);
  auto a = (const float*)c.ptr(1);
  long long n = c.i64(2);
  if (c.failed) return nullptr;
  return check(env, c, ns2_accumulate(y, a, n));
}

// addRows(a, b, y, rows, n)
napi_value AddRows(napi_env env, napi_callback_info info) {
  ARGS(5);
  auto a = (const float*)c.ptr(0);
  auto b = (const float*)c.ptr(1);
  auto y = (float*)c.ptr(2);
  int rows = c.i32(3), n = c.i32(4);
  if (c.failed) return nullptr;
  return check(env, c, ns2_add_rows(a, b, y, rows, n));
}

// rowSum(x, w, y, rows, N, scale)
napi_value RowSum(napi_env env, napi_callback_info info) {
  ARGS(6);
  auto x = (const float*)c.ptr(0);
  auto w = (const float*)c.ptr(1);
  auto y = (float*)c.ptr(2);
  int rows = c.i32(3), N = c.i32(4);
  float s = c.f32(5);
  if (c.failed) return nullptr;
  return check(env, c, ns2_row_sum(x, w, y, rows, N, s));
}

// rmsnorm(x, w, y, rows, cols, eps)
napi_value Rmsnorm(napi_env env, napi_callback_info info) {
  ARGS(6);
  auto x = (const float*)c.ptr(0);
  auto w = (const float*)c.ptr(1);
  auto y = (float*)c.ptr(2);
  int rows = c.i32(3), cols = c.i32(4);
  float eps = c.f32(5);
  if (c.failed) return nullptr;
  return check(env, c, ns2_rmsnorm(x, w, y, rows, cols, eps));
}

// transpose(x, y, rows, cols)
napi_value Transpose(napi_env env, napi_callback_info info) {
  ARGS(4);
  auto x = (const float*)c.ptr(0);
  auto y = (float*)c.ptr(1);
  int rows = c.i32(2), cols = c.i32(3);
  if (c.failed) return nullptr;
  return check(env, c, ns2_transpose(x, y, rows, cols));
}

// addRmsnorm(x, a, wAdd, wOut, y, rows, cols, eps)
napi_value AddRmsnorm(napi_env env, napi_callback_info info) {
  ARGS(8);
  auto x = (float*)c.ptr(0);
  auto a = (const float*)c.ptr(1);
  auto wa = (const float*)c.ptr(2);
  auto wo = (const float*)c.ptr(3);
  auto y = (float*)c.ptr(4);
  int rows = c.i32(5), cols = c.i32(6);
  float eps = c.f32(7);
  if (c.failed) return nullptr;
  return check(env, c, ns2_add_rmsnorm(x, a, wa, wo, y, rows, cols, eps));
}

// linearBf16Glu(A, lda, W, bias, Y, M, N, K, act)
napi_value LinearBf16Glu(napi_env env, napi_callback_info info) {
  ARGS(9);
  auto A = (const float*)c.ptr(0);
  int lda = c.i32(1);
  auto W = (const uint16_t*)c.ptr(2);
  auto bias = (const float*)c.ptr(3);
  auto Y = (float*)c.ptr(4);
  int M = c.i32(5), N = c.i32(6), K = c.i32(7), act = c.i32(8);
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_bf16_glu(A, lda, W, bias, Y, M, N, K, act));
}

// linearBf16HeadNorm(A, lda, W, bias, C, M, N, K, w1, H1, w2, H2, D, cs, sinOff, ropeRows, eps)
napi_value LinearBf16HeadNorm(napi_env env, napi_callback_info info) {
  ARGS(17);
  auto A = (const float*)c.ptr(0);
  int lda = c.i32(1);
  auto W = (const uint16_t*)c.ptr(2);
  auto bias = (const float*)c.ptr(3);
  auto C = (float*)c.ptr(4);
  int M = c.i32(5), N = c.i32(6), K = c.i32(7);
  auto w1 = (const float*)c.ptr(8);
  int H1 = c.i32(9);
  auto w2 = (const float*)c.ptr(10);
  int H2 = c.i32(11), D = c.i32(12);
  auto cs = (const float*)c.ptr(13);
  long long sinOff = c.i64(14);
  int ropeRows = c.i32(15);
  float eps = c.f32(16);
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_bf16_head_norm(A, lda, W, bias, C, M, N, K, w1, H1, w2, H2, D, cs, sinOff, ropeRows, eps));
}

// linearBf16HeadNormF16kv(A, lda, W, bias, C, M, N, K, w1, H1, w2, H2, D, cs, sinOff, ropeRows, eps, kv16, ldkv)
napi_value LinearBf16HeadNormF16kv(napi_env env, napi_callback_info info) {
  ARGS(19);
  auto A = (const float*)c.ptr(0);
  int lda = c.i32(1);
  auto W = (const uint16_t*)c.ptr(2);
  auto bias = (const float*)c.ptr(3);
  auto C = (float*)c.ptr(4);
  int M = c.i32(5), N = c.i32(6), K = c.i32(7);
  auto w1 = (const float*)c.ptr(8);
  int H1 = c.i32(9);
  auto w2 = (const float*)c.ptr(10);
  int H2 = c.i32(11), D = c.i32(12);
  auto cs = (const float*)c.ptr(13);
  long long sinOff = c.i64(14);
  int ropeRows = c.i32(15);
  float eps = c.f32(16);
  auto kv16 = (uint16_t*)c.ptr(17);
  int ldkv = c.i32(18);
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_bf16_head_norm_f16kv(A, lda, W, bias, C, M, N, K, w1, H1, w2, H2, D, cs, sinOff,
                                                       ropeRows, eps, kv16, ldkv));
}

// linearBf16GluDown(A, lda, W, bias, M, N, K, act, wdTiled, Nd, part)
napi_value LinearBf16GluDown(napi_env env, napi_callback_info info) {
  ARGS(11);
  auto A = (const float*)c.ptr(0);
  int lda = c.i32(1);
  auto W = (const uint16_t*)c.ptr(2);
  auto bias = (const float*)c.ptr(3);
  int M = c.i32(4), N = c.i32(5), K = c.i32(6), act = c.i32(7);
  auto wd = (const uint16_t*)c.ptr(8);
  int Nd = c.i32(9);
  auto part = (float*)c.ptr(10);
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_bf16_glu_down(A, lda, W, bias, M, N, K, act, wd, Nd, part));
}

// partsAddRmsnormTiled(part, splits, bias, x, wAdd, wOut, yt, M, N, eps)
napi_value PartsAddRmsnormTiled(napi_env env, napi_callback_info info) {
  ARGS(10);
  auto part = (const float*)c.ptr(0);
  int splits = c.i32(1);
  auto bias = (const float*)c.ptr(2);
  auto x = (float*)c.ptr(3);
  auto wAdd = (const float*)c.ptr(4);
  auto wOut = (const float*)c.ptr(5);
  auto yt = (uint16_t*)c.ptr(6);
  int M = c.i32(7), N = c.i32(8);
  float eps = c.f32(9);
  if (c.failed) return nullptr;
  return check(env, c, ns2_parts_add_rmsnorm_tiled(part, splits, bias, x, wAdd, wOut, yt, M, N, eps));
}

// linearF16wTiledHeadNormF16kv(At, Wt, bias, C, M, N, K, w1, H1, w2, H2, D, cs, sinOff, ropeRows, eps, kv16, ldkv)
napi_value LinearF16wTiledHeadNormF16kv(napi_env env, napi_callback_info info) {
  ARGS(18);
  auto At = (const uint16_t*)c.ptr(0);
  auto Wt = (const uint16_t*)c.ptr(1);
  auto bias = (const float*)c.ptr(2);
  auto C = (float*)c.ptr(3);
  int M = c.i32(4), N = c.i32(5), K = c.i32(6);
  auto w1 = (const float*)c.ptr(7);
  int H1 = c.i32(8);
  auto w2 = (const float*)c.ptr(9);
  int H2 = c.i32(10), D = c.i32(11);
  auto cs = (const float*)c.ptr(12);
  long long sinOff = c.i64(13);
  int ropeRows = c.i32(14);
  float eps = c.f32(15);
  auto kv16 = (uint16_t*)c.ptr(16);
  int ldkv = c.i32(17);
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_f16w_tiled_head_norm_f16kv(At, Wt, bias, C, M, N, K, w1, H1, w2, H2, D, cs, sinOff,
                                                             ropeRows, eps, kv16, ldkv));
}

// linearF16wTiledGluDown(At, Wt, bias, M, N, K, act, wdTiled, Nd, part)
napi_value LinearF16wTiledGluDown(napi_env env, napi_callback_info info) {
  ARGS(10);
  auto At = (const uint16_t*)c.ptr(0);
  auto Wt = (const uint16_t*)c.ptr(1);
  auto bias = (const float*)c.ptr(2);
  int M = c.i32(3), N = c.i32(4), K = c.i32(5), act = c.i32(6);
  auto wd = (const uint16_t*)c.ptr(7);
  int Nd = c.i32(8);
  auto part = (float*)c.ptr(9);
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_f16w_tiled_glu_down(At, Wt, bias, M, N, K, act, wd, Nd, part));
}

// linearBf16AddRmsnorm(A, lda, W, bias, x, wAdd, wOut, y, M, N, K, eps)
napi_value LinearBf16AddRmsnorm(napi_env env, napi_callback_info info) {
  ARGS(12);
  auto A = (const float*)c.ptr(0);
  int lda = c.i32(1);
  auto W = (const uint16_t*)c.ptr(2);
  auto bias = (const float*)c.ptr(3);
  auto x = (float*)c.ptr(4);
  auto wa = (const float*)c.ptr(5);
  auto wo = (const float*)c.ptr(6);
  auto y = (float*)c.ptr(7);
  int M = c.i32(8), N = c.i32(9), K = c.i32(10);
  float eps = c.f32(11);
  if (c.failed) return nullptr;
  return check(env, c, ns2_linear_bf16_add_rmsnorm(A, lda, W, bias, x, wa, wo, y, M, N, K, eps));
}

napi_value Module(napi_env env, napi_value exports) {
  struct Fn {
    const char* name;
    napi_callback cb;
  } fns[] = {
      {"init", Init}, {"deviceInfo", DeviceInfo}, {"malloc", Malloc}, {"free", Free},
      {"poolRound", PoolRound}, {"poolGet", PoolGet}, {"poolPut", PoolPut}, {"poolTrim", PoolTrim},
      {"poolStats", PoolStats}, {"h2d", H2D}, {"d2h", D2H}, {"sync", Sync}, {"fill", Fill},
      {"eventCreate", EventCreate}, {"eventRecord", EventRecord}, {"eventElapsed", EventElapsed},
      {"eventDestroy", EventDestroy}, {"graphBegin", GraphBegin}, {"graphEnd", GraphEnd},
      {"graphLaunch", GraphLaunch}, {"graphDestroy", GraphDestroy}, {"profileEnable", ProfileEnable}, {"profileReset", ProfileReset},
      {"profileReport", ProfileReport}, {"hadamard256", Hadamard256}, {"rotateF16", RotateF16},
      {"tileI8Weight", TileI8Weight}, {"linearI8Tiled", LinearI8Tiled},
      {"tileI8WeightGlu", TileI8WeightGlu}, {"linearI8GluRotTiled", LinearI8GluRotTiled},
      {"tileBf16Weight", TileBf16Weight}, {"linearF16wTiled", LinearF16wTiled}, {"toTiledF16", ToTiledF16},
      {"normModF16", NormModF16},
      {"linearI8", LinearI8}, {"linearBf16", LinearBf16}, {"attention", Attention},
      {"attentionRows", AttentionRows}, {"attentionRowsF16kv", AttentionRowsF16kv},
      {"attentionRowsF16kvOproj", AttentionRowsF16kvOproj}, {"partsAddRmsnorm", PartsAddRmsnorm}, {"attentionText", AttentionText},
      {"linearI8TiledVpack", LinearI8TiledVpack}, {"attentionVpackBytes", AttentionVpackBytes},
      {"attentionVpacked", AttentionVpacked},
      {"headNorm", HeadNorm}, {"headNorm2", HeadNorm2}, {"normMod", NormModT<false>}, {"normModRotateF16", NormModT<true>},
      {"glu", GluT<false>}, {"gluRotateF16", GluT<true>}, {"elementwise", Elementwise},
      {"accumulate", Accumulate}, {"addRows", AddRows}, {"rowSum", RowSum}, {"rmsnorm", Rmsnorm},
      {"addRmsnorm", AddRmsnorm}, {"linearBf16AddRmsnorm", LinearBf16AddRmsnorm},
      {"linearBf16Glu", LinearBf16Glu}, {"linearBf16GluDown", LinearBf16GluDown},
      {"partsAddRmsnormTiled", PartsAddRmsnormTiled}, {"linearF16wTiledHeadNormF16kv", LinearF16wTiledHeadNormF16kv},
      {"linearF16wTiledGluDown", LinearF16wTiledGluDown}, {"linearBf16HeadNorm", LinearBf16HeadNorm},
      {"linearBf16HeadNormF16kv", LinearBf16HeadNormF16kv}, {"transpose", Transpose},
  };
  for (const Fn& f : fns) {
    napi_value fn;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn);
    napi_set_named_property(env, exports, f.name, fn);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Module)
