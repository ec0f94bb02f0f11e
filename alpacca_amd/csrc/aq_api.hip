// aq_api.hip - the C ABI (include/alpacca_amd.h): matrix upload to HBM,
// argument validation with the reference's error classes, host<->device
// staging for callers that pass host pointers, and kernel dispatch.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <set>
#include <utility>
#include <new>
#include <vector>

#include "aq_internal.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

// set when workspace() refused to grow a stream's scratch under graph capture
thread_local bool g_ws_refused_capture = false;

int hip_fail(hipError_t e, const char *what) {
  if (g_ws_refused_capture) {
    g_ws_refused_capture = false;
    return fail(AQ_ERR_RUNTIME,
                "%s: the library's scratch for this stream is too small and the stream is "
                "capturing a graph (no device allocation under capture): run the call once "
                "eagerly before capture, or use an allocation-free entry point", what);
  }
  return fail(AQ_ERR_RUNTIME, "%s: %s", what, hipGetErrorString(e));
}

#define AQ_HIP(call, what)                 \
  do {                                     \
    hipError_t e_ = (call);                \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

struct Geom {
  int dtype, block_elems, block_bytes, sub_len, affine;
};
// QUANT_GEOMETRY of alpacca/quants.py:317-326
const Geom kGeom[] = {
    {AQ_Q8_0, 32, 34, 32, 0},   {AQ_Q4_0, 32, 18, 32, 0},
    {AQ_Q4_1, 32, 20, 32, 1},   {AQ_Q5_0, 32, 22, 32, 0},
    {AQ_Q5_1, 32, 24, 32, 1},   {AQ_Q4_K, 256, 144, 32, 1},
    {AQ_Q5_K, 256, 176, 32, 1}, {AQ_Q6_K, 256, 210, 16, 0},
};
// dense matrices: 32 values per block along K (F32 128 B, F16/BF16 64 B)
const Geom kDenseGeom[] = {
    {AQ_F32, 32, 128, 32, 0}, {AQ_F16, 32, 64, 32, 0}, {AQ_BF16, 32, 64, 32, 0}};
const Geom *find_geom(int dtype, bool dense_too = false) {
  for (const Geom &g : kGeom)
    if (g.dtype == dtype) return &g;
  if (dense_too)
    for (const Geom &g : kDenseGeom)
      if (g.dtype == dtype) return &g;
  return nullptr;
}

const char *dtype_name(int dtype) {
  switch (dtype) {
    case AQ_Q8_0: return "Q8_0";
    case AQ_Q4_0: return "Q4_0";
    case AQ_Q4_1: return "Q4_1";
    case AQ_Q5_0: return "Q5_0";
    case AQ_Q5_1: return "Q5_1";
    case AQ_Q4_K: return "Q4_K";
    case AQ_Q5_K: return "Q5_K";
    case AQ_Q6_K: return "Q6_K";
    case AQ_F32: return "F32";
    case AQ_F16: return "F16";
    case AQ_BF16: return "BF16";
    default: return "?";
  }
}

// Field table (raw offset, bytes) per dtype, from the format structs.
struct FieldList {
  int n;
  aq::FieldSpec f[4];
  bool raw_ok;
};
template <class F>
FieldList fields_of() {
  FieldList L{F::NPL, {}, F::RAW_OK};
  for (int i = 0; i < F::NPL; ++i) L.f[i] = F::FIELDS[i];
  return L;
}
bool field_list(int dtype, FieldList &out) {
  switch (dtype) {
    case AQ_Q4_K: out = fields_of<aq::Q4K>(); return true;
    case AQ_Q5_K: out = fields_of<aq::Q5K>(); return true;
    case AQ_Q6_K: out = fields_of<aq::Q6K>(); return true;
    case AQ_Q8_0: out = fields_of<aq::Q80>(); return true;
    case AQ_Q4_0: out = fields_of<aq::Q40>(); return true;
    case AQ_Q4_1: out = fields_of<aq::Q41>(); return true;
    case AQ_Q5_0: out = fields_of<aq::Q50>(); return true;
    case AQ_Q5_1: out = fields_of<aq::Q51>(); return true;
    case AQ_F32: out = fields_of<aq::F32D>(); return true;
    case AQ_F16: out = fields_of<aq::F16D>(); return true;
    case AQ_BF16: out = fields_of<aq::BF16D>(); return true;
    default: return false;
  }
}

// ---- devices ---------------------------------------------------------------
constexpr int kMaxDev = 64;
aq::DeviceInfo g_dev[kMaxDev];
bool g_dev_ok[kMaxDev];
std::mutex g_dev_mu;

int ensure_device(int device) {
  if (device < 0 || device >= kMaxDev)
    return fail(AQ_ERR_VALUE, "device %d out of range", device);
  std::lock_guard<std::mutex> lk(g_dev_mu);
  if (g_dev_ok[device]) return AQ_OK;
  int n = 0;
  AQ_HIP(hipGetDeviceCount(&n), "hipGetDeviceCount");
  if (device >= n)
    return fail(AQ_ERR_RUNTIME, "HIP device %d not present (%d visible)",
                device, n);
  hipDeviceProp_t prop;
  AQ_HIP(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  g_dev[device].cus = prop.multiProcessorCount;
  size_t lds = prop.sharedMemPerBlockOptin ? prop.sharedMemPerBlockOptin
                                           : prop.sharedMemPerBlock;
  g_dev[device].lds_max = lds;
  g_dev_ok[device] = true;
  return AQ_OK;
}

int current_device(int &dev) {
  AQ_HIP(hipGetDevice(&dev), "hipGetDevice");
  return ensure_device(dev);
}

int noalloc_scratch(int device, float **out);  // the static scratch (below)

// ---- per-thread device staging for host-pointer callers ------------------
struct Staging {
  void *ptr = nullptr;
  size_t cap = 0;
  int device = -1;
};
thread_local Staging g_stage[3];  // 0: input, 1: output, 2: indices

int stage_buffer(int which, size_t bytes, int device, void **out) {
  Staging &s = g_stage[which];
  if (s.ptr && (s.cap < bytes || s.device != device)) {
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(s.device);
    (void)hipFree(s.ptr);
    (void)hipSetDevice(prev);
    s.ptr = nullptr;
    s.cap = 0;
  }
  if (!s.ptr) {
    size_t cap = bytes < 4096 ? 4096 : bytes;
    cap = (cap + 4095) & ~(size_t)4095;
    AQ_HIP(hipMalloc(&s.ptr, cap), "hipMalloc(staging)");
    s.cap = cap;
    s.device = device;
  }
  *out = s.ptr;
  return AQ_OK;
}

// Per-thread pinned host buffers (0: input, 1: output) between the caller's
// arrays and the device: a copy from or to pageable memory goes through the
// runtime's own bounce buffer and costs ~15 us a side, pinned memory is read
// and written by kernels directly.
struct PinStaging {
  void *ptr = nullptr;
  size_t cap = 0;
};
thread_local PinStaging g_pin[2];

int pin_buffer(int which, size_t bytes, void **out) {
  PinStaging &p = g_pin[which];
  if (p.ptr && p.cap < bytes) {
    (void)hipHostFree(p.ptr);
    p.ptr = nullptr;
    p.cap = 0;
  }
  if (!p.ptr) {
    size_t cap = (size_t)1 << 16;
    while (cap < bytes) cap <<= 1;
    AQ_HIP(hipHostMalloc(&p.ptr, cap, hipHostMallocDefault), "hipHostMalloc(staging)");
    p.cap = cap;
  }
  *out = p.ptr;
  return AQ_OK;
}

// n 4-byte words from src to dst (a kernel reading pinned host memory: no
// copy-engine round trip for the small inputs of a call)
__global__ void k_copy_words(const uint32_t *__restrict__ src, uint32_t *__restrict__ dst,
                             int64_t n) {
  const int64_t n4 = n / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t i = t; i < n4; i += stride)
    reinterpret_cast<uint4 *>(dst)[i] = reinterpret_cast<const uint4 *>(src)[i];
  for (int64_t i = 4 * n4 + t; i < n; i += stride) dst[i] = src[i];
}

// Inputs and outputs up to this size are copied by k_copy_words (coalesced
// reads or writes of pinned memory); larger ones go through the copy engine.
constexpr size_t kDirectBytes = (size_t)1 << 20;

}  // namespace

namespace {

// Shared wrapper: stage a host input/output if needed, run `launch`, copy the
// output back and wait when the caller gave a host output pointer.  Host data
// passes through per-thread pinned buffers; a small input is copied to the
// device by a kernel, a small output is written into pinned memory by a copy
// kernel, or, with `out_direct` (a launch that only stores its output, once
// per element), by the call's own kernels (a matvec called on host arrays:
// ~15 us against ~30 us through pageable copies).
template <class Launch>
int run_staged(const aq_matrix *m, const void *in, size_t in_bytes,
                      void *outp, size_t out_bytes, int flags, void *stream,
                      Launch launch, bool out_direct = false) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  int prev = 0;
  AQ_HIP(hipGetDevice(&prev), "hipGetDevice");
  if (prev != m->device) AQ_HIP(hipSetDevice(m->device), "hipSetDevice");
  const void *din = in;
  void *dout = outp;
  int rc = AQ_OK;
  hipError_t e = hipSuccess;
  void *pin_out = nullptr;
  const bool direct_out = out_bytes <= kDirectBytes;
  if (!(flags & AQ_IN_DEVICE) && in_bytes) {
    void *buf = nullptr, *pin = nullptr;
    rc = stage_buffer(0, in_bytes, m->device, &buf);
    if (!rc) rc = pin_buffer(0, in_bytes, &pin);
    if (!rc) {
      memcpy(pin, in, in_bytes);
      if (in_bytes <= kDirectBytes && in_bytes % 4 == 0) {
        const int64_t words = (int64_t)(in_bytes / 4);
        const int64_t wg = std::min<int64_t>((words / 4 + 255) / 256 + 1, 64);
        hipLaunchKernelGGL(k_copy_words, dim3((unsigned)wg), dim3(256), 0, s,
                           static_cast<const uint32_t *>(pin), static_cast<uint32_t *>(buf),
                           words);
        e = hipGetLastError();
        if (e != hipSuccess) rc = hip_fail(e, "input copy launch");
      } else {
        e = hipMemcpyAsync(buf, pin, in_bytes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) rc = hip_fail(e, "hipMemcpyAsync(H2D)");
      }
      din = buf;
    }
  }
  // the launch writes straight into pinned memory: small outputs that it
  // only stores (no copy kernel behind it)
  const bool to_pinned = out_direct && direct_out && out_bytes % 4 == 0;
  if (!rc && !(flags & AQ_OUT_DEVICE) && out_bytes) {
    void *buf = nullptr;
    rc = pin_buffer(1, out_bytes, &pin_out);
    if (!rc && !to_pinned) rc = stage_buffer(1, out_bytes, m->device, &buf);
    dout = to_pinned ? pin_out : buf;
  }
  if (!rc && out_bytes) {
    e = launch(din, dout, s);
    if (e != hipSuccess) rc = hip_fail(e, "kernel launch");
  }
  if (!rc && !(flags & AQ_OUT_DEVICE) && out_bytes && !to_pinned) {
    if (direct_out && out_bytes % 4 == 0) {  // coalesced kernel writes into pinned memory
      const int64_t words = (int64_t)(out_bytes / 4);
      const int64_t wg = std::min<int64_t>((words / 4 + 255) / 256 + 1, 64);
      hipLaunchKernelGGL(k_copy_words, dim3((unsigned)wg), dim3(256), 0, s,
                         static_cast<const uint32_t *>(dout), static_cast<uint32_t *>(pin_out),
                         words);
      e = hipGetLastError();
      if (e != hipSuccess) rc = hip_fail(e, "output copy launch");
    } else {
      e = hipMemcpyAsync(pin_out, dout, out_bytes, hipMemcpyDeviceToHost, s);
      if (e != hipSuccess) rc = hip_fail(e, "hipMemcpyAsync(D2H)");
    }
  }
  // a call that staged either side waits for its work: the thread's staging
  // buffers are reused by its next call, on whatever stream that runs
  const bool staged = (!(flags & AQ_IN_DEVICE) && in_bytes) ||
                      (!(flags & AQ_OUT_DEVICE) && out_bytes);
  if (!rc && staged) {
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
  }
  if (!rc && !(flags & AQ_OUT_DEVICE) && out_bytes) memcpy(outp, pin_out, out_bytes);
  if (prev != m->device) (void)hipSetDevice(prev);
  return rc;
}

__global__ void k_fill_zero(float *p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}
hipError_t fill_zero(float *p, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, s, p, n);
  return hipGetLastError();
}

// Column slices for a matvec whose rows are wider than one launch can stage
// x for: nb_row blocks cut into the fewest windows of at most kmax columns,
// as even as whole blocks allow, in K order.  y = sum of the windows'
// products, added one window after the other (a fixed order).
struct ColSlice {
  int64_t nb0, nb;
};
std::vector<ColSlice> column_slices(int64_t nb_row, int64_t block_elems, int64_t kmax) {
  const int64_t max_nb = kmax / block_elems;
  const int64_t n = (nb_row + max_nb - 1) / max_nb;
  std::vector<ColSlice> out;
  for (int64_t i = 0, nb0 = 0; i < n; ++i) {
    const int64_t nb = (nb_row - nb0 + (n - i) - 1) / (n - i);
    out.push_back({nb0, nb});
    nb0 += nb;
  }
  return out;
}

}  // namespace

namespace aq {
const DeviceInfo &device_info(int device) { return g_dev[device]; }

namespace {
struct WsEntry {
  int device;
  hipStream_t stream;
  void *ptr;
  size_t bytes;
  bool captured;  // handed out while the stream was capturing a graph
};
std::mutex g_ws_mu;
std::vector<WsEntry> g_ws_live;     // one buffer per (device, stream)
std::vector<void *> g_ws_retired;   // buffers a captured graph may still use

bool stream_capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}
// Give up e's buffer: freed once the stream's queued work is done, or kept
// for the life of the process when a captured graph may refer to it.
void ws_drop(WsEntry &e, bool capturing_now) {
  if (!e.ptr) return;
  if (e.captured || capturing_now) {
    g_ws_retired.push_back(e.ptr);
  } else {
    (void)hipStreamSynchronize(e.stream);
    (void)hipFree(e.ptr);
  }
  e.ptr = nullptr;
  e.bytes = 0;
  e.captured = false;
}
}  // namespace

void *workspace(int device, hipStream_t s, size_t bytes) {
  // sizes grow geometrically (powers of two from 1 MiB), so a run of
  // growing requests allocates O(log) times and holds < 2x the largest
  size_t cap = (size_t)1 << 20;
  while (cap < bytes) cap <<= 1;
  // Under graph capture nothing is allocated (hipMalloc is not a capturable
  // operation): the stream's buffer must already be large enough, from an
  // eager call of the same shape before capture.  The buffer a capture
  // hands out is kept for the process's life once it is outgrown or
  // released, since the graph may still be replayed.
  const bool capturing = stream_capturing(s);
  std::lock_guard<std::mutex> lock(g_ws_mu);
  for (WsEntry &e : g_ws_live) {
    if (e.device != device || e.stream != s) continue;
    if (e.bytes < bytes) {
      if (capturing) {
        g_ws_refused_capture = true;
        return nullptr;
      }
      ws_drop(e, false);
      if (hipMalloc(&e.ptr, cap) != hipSuccess) return e.ptr = nullptr;
      e.bytes = cap;
    }
    e.captured = e.captured || capturing;
    return e.ptr;
  }
  if (capturing) {
    g_ws_refused_capture = true;
    return nullptr;
  }
  void *p = nullptr;
  if (hipMalloc(&p, cap) != hipSuccess) return nullptr;
  g_ws_live.push_back({device, s, p, cap, false});
  return p;
}

void release_workspace(hipStream_t s) {
  std::lock_guard<std::mutex> lock(g_ws_mu);
  for (size_t i = 0; i < g_ws_live.size();) {
    if (g_ws_live[i].stream == s) {
      int prev = 0;
      (void)hipGetDevice(&prev);
      (void)hipSetDevice(g_ws_live[i].device);
      ws_drop(g_ws_live[i], false);
      (void)hipSetDevice(prev);
      g_ws_live.erase(g_ws_live.begin() + i);
    } else {
      ++i;
    }
  }
}

hipError_t set_dynamic_lds(const void *kern, int bytes) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  static std::mutex mu;
  static std::set<std::pair<const void *, int>> done;
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({kern, device})) return hipSuccess;
  e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.insert({kern, device});
  return e;
}
}  // namespace aq

namespace {
// Status of an attention launch: the launchers refuse (hipErrorInvalidValue)
// a scratch smaller than the partials their grid writes, which is a sizing
// mistake of the caller, reported as such.
int attention_status(hipError_t e, int n_kv, int head_dim, int group, int64_t n_ctx,
                     int64_t T, size_t capacity) {
  if (e == hipSuccess) return AQ_OK;
  const size_t need = aq::attention_launch_extent_bytes(n_kv, head_dim, group, n_ctx, T);
  if (e == hipErrorInvalidValue && need > capacity)
    return fail(AQ_ERR_VALUE, "attention partials of this launch need %zu bytes, more than "
                "the %zu-byte scratch", need, capacity);
  return hip_fail(e, "attention launch");
}
}  // namespace

extern "C" {

const char *aq_version(void) { return "alpacca_amd 0.1.0 (gfx950)"; }

const char *aq_last_error(void) { return g_err; }

int aq_device_count(int *count) {
  if (!count) return fail(AQ_ERR_VALUE, "count is NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) n = 0;
  *count = n;
  return AQ_OK;
}

int aq_init(int device) {
  int rc = ensure_device(device);
  if (rc) return rc;
  AQ_HIP(hipSetDevice(device), "hipSetDevice");
  float *scratch_ptr = nullptr;  // the static scratch's address on this device
  return noalloc_scratch(device, &scratch_ptr);
}

int aq_geometry(int dtype, int *block_elems, int *block_bytes, int *sub_len,
                int *affine) {
  const Geom *g = find_geom(dtype);
  if (!g) return fail(AQ_ERR_VALUE, "quantized matvec does not support dtype %d", dtype);
  if (block_elems) *block_elems = g->block_elems;
  if (block_bytes) *block_bytes = g->block_bytes;
  if (sub_len) *sub_len = g->sub_len;
  if (affine) *affine = g->affine;
  return AQ_OK;
}

int aq_matrix_create(const void *blocks, size_t nbytes, int dtype, int64_t rows,
                     int64_t cols, int layout, aq_matrix **out) {
  if (!out) return fail(AQ_ERR_VALUE, "out is NULL");
  *out = nullptr;
  const Geom *g = find_geom(dtype, true);
  if (!g)
    return fail(AQ_ERR_VALUE, "quantized matvec does not support dtype %d", dtype);
  if (rows < 0 || cols < 0)
    return fail(AQ_ERR_VALUE, "negative shape (%lld, %lld)", (long long)rows,
                (long long)cols);
  if (cols % g->block_elems)
    return fail(AQ_ERR_VALUE, "%s matrix columns must be a multiple of %d",
                dtype_name(dtype), g->block_elems);
  const int64_t nb_row = cols / g->block_elems;
  const size_t expected = (size_t)rows * (size_t)nb_row * (size_t)g->block_bytes;
  if (nbytes != expected)
    return fail(AQ_ERR_VALUE, "%s matrix has %zu bytes, expected %zu",
                dtype_name(dtype), nbytes, expected);
  if (expected && !blocks) return fail(AQ_ERR_VALUE, "blocks is NULL");
  FieldList fl;
  field_list(dtype, fl);
  if (layout == AQ_LAYOUT_AUTO)
    layout = fl.raw_ok ? AQ_LAYOUT_RAW : AQ_LAYOUT_SPLIT;
  if (layout != AQ_LAYOUT_RAW && layout != AQ_LAYOUT_SPLIT)
    return fail(AQ_ERR_VALUE, "unknown layout %d", layout);
  if (layout == AQ_LAYOUT_RAW && !fl.raw_ok)
    return fail(AQ_ERR_VALUE,
                "%s blocks are not 16-byte aligned; use the SPLIT layout",
                dtype_name(dtype));
  int dev = 0;
  int rc = current_device(dev);
  if (rc) return rc;

  aq_matrix *m = new (std::nothrow) aq_matrix();
  if (!m) return fail(AQ_ERR_RUNTIME, "out of host memory");
  m->dtype = dtype;
  m->layout = layout;
  m->device = dev;
  m->rows = rows;
  m->cols = cols;
  m->nb_row = nb_row;
  m->nb_pitch = nb_row;
  m->raw_bytes = expected;
  const size_t nblk = (size_t)rows * (size_t)nb_row;

  // plane sizes, each rounded up to 256 B
  size_t off[4] = {0, 0, 0, 0};
  size_t total = 0;
  if (layout == AQ_LAYOUT_RAW) {
    total = expected;
  } else {
    for (int i = 0; i < fl.n; ++i) {
      off[i] = total;
      total += ((size_t)fl.f[i].bytes * nblk + 255) & ~(size_t)255;
    }
  }
  m->dev_bytes = total < 256 ? 256 : total;
  hipError_t e = hipMalloc(reinterpret_cast<void **>(&m->dev), m->dev_bytes);
  if (e != hipSuccess) {
    delete m;
    return hip_fail(e, "hipMalloc(matrix)");
  }
  const uint8_t *src = static_cast<const uint8_t *>(blocks);
  if (layout == AQ_LAYOUT_RAW) {
    if (expected) e = hipMemcpy(m->dev, src, expected, hipMemcpyHostToDevice);
    for (int i = 0; i < fl.n; ++i) {
      m->planes.p[i] = m->dev + fl.f[i].raw_off;
      m->planes.stride[i] = g->block_bytes;
    }
  } else {
    std::vector<uint8_t> img;
    try {
      img.assign(total, 0);
    } catch (...) {
      (void)hipFree(m->dev);
      delete m;
      return fail(AQ_ERR_RUNTIME, "out of host memory for the repack image");
    }
    for (int i = 0; i < fl.n; ++i) {
      const int fo = fl.f[i].raw_off, fb = fl.f[i].bytes;
      uint8_t *dst = img.data() + off[i];
      for (size_t b = 0; b < nblk; ++b)
        memcpy(dst + b * fb, src + b * g->block_bytes + fo, fb);
      m->planes.p[i] = m->dev + off[i];
      m->planes.stride[i] = fb;
    }
    if (total) e = hipMemcpy(m->dev, img.data(), total, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    (void)hipFree(m->dev);
    delete m;
    return hip_fail(e, "hipMemcpy(matrix upload)");
  }
  *out = m;
  return AQ_OK;
}

int aq_matrix_destroy(aq_matrix *m) {
  if (!m) return AQ_OK;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(m->device);
  hipError_t e = hipFree(m->dev);
  (void)hipSetDevice(prev);
  delete m;
  if (e != hipSuccess) return hip_fail(e, "hipFree(matrix)");
  return AQ_OK;
}

int aq_matrix_info(const aq_matrix *m, int64_t *rows, int64_t *cols, int *dtype,
                   int *layout, size_t *device_bytes) {
  if (!m) return fail(AQ_ERR_VALUE, "matrix is NULL");
  if (rows) *rows = m->rows;
  if (cols) *cols = m->cols;
  if (dtype) *dtype = m->dtype;
  if (layout) *layout = m->layout;
  if (device_bytes) *device_bytes = m->dev_bytes;
  return AQ_OK;
}

int aq_release_workspace(void *stream) {
  aq::release_workspace(static_cast<hipStream_t>(stream));
  return AQ_OK;
}

int aq_synchronize(void *stream) {
  AQ_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)),
         "hipStreamSynchronize");
  return AQ_OK;
}

int aq_matvec(const aq_matrix *m, const float *x, float *y, int flags,
              void *stream) {
  if (!m) return fail(AQ_ERR_VALUE, "matrix is NULL");
  if ((m->cols && !x) || (m->rows && !y))
    return fail(AQ_ERR_VALUE, "x / y is NULL");
  // dense matrices have no integer kernel
  const bool fp32 = (flags & AQ_MATVEC_FP32) != 0 || aq::is_dense(m->dtype);
  // x is staged in LDS; wider rows run as column windows of at most kmax
  // columns whose products are added in K order
  const int64_t kmax = fp32 ? aq::matvec_max_cols(m->dtype, m->device)
                            : aq::matvec_i8_max_cols(m->dtype, m->device);
  if (!fp32 && m->rows >= INT32_MAX)
    return fail(AQ_ERR_VALUE, "matvec supports at most 2^31 - 2 rows per call");
  const int64_t be = m->nb_row ? m->cols / m->nb_row : 1;
  if (kmax < be) return fail(AQ_ERR_RUNTIME, "device LDS too small for one block of x");
  return run_staged(
      m, x, (size_t)m->cols * 4, y, (size_t)m->rows * 4, flags, stream,
      [&](const void *din, void *dout, hipStream_t s) {
        const float *xin = static_cast<const float *>(din);
        float *yout = static_cast<float *>(dout);
        if (m->cols == 0) return fill_zero(yout, m->rows, s);
        if (m->cols <= kmax)
          return fp32 ? aq::launch_matvec(m, xin, yout, s)
                      : aq::launch_matvec_i8(m, xin, yout, s);
        hipError_t e = hipSuccess;
        bool first = true;
        for (const ColSlice &c : column_slices(m->nb_row, be, kmax)) {
          const aq_matrix v = aq::column_window(*m, c.nb0, c.nb);
          const float *xs = xin + c.nb0 * be;
          if (fp32) {
            e = aq::launch_matvec(&v, xs, yout, s, !first);
          } else {
            aq::MatvecFusion fu{};
            fu.accumulate = !first;
            const aq_matrix *pv = &v;
            e = aq::launch_matvec_i8_multi(&pv, 1, xs, &yout, s, &fu);
          }
          if (e != hipSuccess) return e;
          first = false;
        }
        return e;
      },
      m->cols <= kmax);  // one launch that stores y once: y may be pinned host memory
}

namespace {
int matvec_multi_impl(const aq_matrix *const *ms, int n, const float *x,
                      float *const *ys, int flags, void *stream,
                      const aq::MatvecFusion *fu, const char *name) {
  if (!ms || !ys || n < 1 || n > 8)
    return fail(AQ_ERR_VALUE, "%s takes 1..8 matrices", name);
  if ((flags & (AQ_IN_DEVICE | AQ_OUT_DEVICE)) != (AQ_IN_DEVICE | AQ_OUT_DEVICE))
    return fail(AQ_ERR_VALUE, "%s needs device x and y pointers", name);
  if (flags & AQ_MATVEC_FP32)
    return fail(AQ_ERR_VALUE, "%s runs the integer kernel only", name);
  // one dtype (and layout) for all matrices, or two: the matrices of the
  // first dtype, then those of a second one that may share the launch
  // (aq::matvec_mixed_supported: K-quant pairs of equal block size)
  int n1 = n;
  for (int i = 0; i < n; ++i) {
    if (!ms[i] || (ms[i]->rows && !ys[i]))
      return fail(AQ_ERR_VALUE, "matrix %d or its output is NULL", i);
    if (aq::is_dense(ms[i]->dtype))
      return fail(AQ_ERR_VALUE, "%s: %s matrices run aq_matvec (fp32 kernel) only", name,
                  dtype_name(ms[i]->dtype));
    if (n1 == n && ms[i]->dtype != ms[0]->dtype) n1 = i;
    const aq_matrix *ref = ms[i < n1 ? 0 : n1];
    if (ms[i]->dtype != ref->dtype || ms[i]->cols != ms[0]->cols ||
        ms[i]->layout != ref->layout || ms[i]->device != ms[0]->device)
      return fail(AQ_ERR_VALUE,
                  "%s: matrix %d differs in dtype, cols, layout "
                  "or device from the matrices before it", name, i);
  }
  if (fu && fu->swiglu_pairs) {
    if (n1 < n) return fail(AQ_ERR_VALUE, "%s: gate/up pairs take one dtype", name);
    if (!aq::matvec_pair_rows(ms[0]->dtype, ms[0]->nb_row))
      return fail(AQ_ERR_VALUE, "%s: gate/up pairs need rows of at most 32 lane units "
                  "(%s K = %lld is too wide)", name, dtype_name(ms[0]->dtype),
                  (long long)ms[0]->cols);
    for (int i = 0; i < n; ++i)
      if (ms[i]->rows % 2)
        return fail(AQ_ERR_VALUE, "%s: gate/up pairs need an even row count", name);
  }
  if (n1 < n && (!aq::matvec_mixed_supported(ms[0]->dtype, ms[n1]->dtype) ||
                 (fu && fu->mode == aq::MatvecFusion::kSwiglu)))
    return fail(AQ_ERR_VALUE, "%s: %s and %s matrices cannot share a launch%s", name,
                dtype_name(ms[0]->dtype), dtype_name(ms[n1]->dtype),
                fu && fu->mode == aq::MatvecFusion::kSwiglu ? " with a SwiGLU input" : "");
  const aq_matrix *m = ms[0];
  if (m->cols && !x) return fail(AQ_ERR_VALUE, "x is NULL");
  int64_t total_rows = 0;
  for (int i = 0; i < n; ++i) total_rows += ms[i]->rows;
  if (total_rows >= INT32_MAX)
    return fail(AQ_ERR_VALUE, "matvec supports at most 2^31 - 2 rows per call");
  // rows wider than one launch stages x for run as column windows (the
  // products added in K order); RMSNorm needs all of x in every launch
  int64_t kmax = INT64_MAX;
  for (int i = 0; i < n; i += (n1 < n ? n1 : n))
    kmax = std::min(kmax, aq::matvec_i8_max_cols(ms[i]->dtype, m->device));
  const bool windows = m->cols > kmax;
  if (windows && fu && fu->mode == aq::MatvecFusion::kNorm)
    return fail(AQ_ERR_VALUE,
                "%s: RMSNorm-staged %s matvec supports at most %lld columns", name,
                dtype_name(m->dtype), (long long)kmax);
  if (windows && fu && fu->swiglu_pairs)
    return fail(AQ_ERR_VALUE, "%s: gate/up pairs need rows of at most 32 lane units", name);
  int prev = 0;
  AQ_HIP(hipGetDevice(&prev), "hipGetDevice");
  if (prev != m->device) AQ_HIP(hipSetDevice(m->device), "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  if (m->cols == 0) {
    // W x_eff = 0: y is zeroed, or left as it is when accumulating
    for (int i = 0; i < n && e == hipSuccess && !(fu && fu->accumulate); ++i)
      e = fill_zero(ys[i], fu && fu->swiglu_pairs ? ms[i]->rows / 2 : ms[i]->rows, s);
  } else if (!windows) {
    e = aq::launch_matvec_i8_multi(ms, n, x, ys, s, fu);
  } else {
    const int64_t be = m->cols / m->nb_row;
    if (kmax < be) {
      if (prev != m->device) (void)hipSetDevice(prev);
      return fail(AQ_ERR_RUNTIME, "device LDS too small for one block of x");
    }
    bool first = true;
    for (const ColSlice &c : column_slices(m->nb_row, be, kmax)) {
      aq_matrix views[8];
      const aq_matrix *pv[8];
      for (int i = 0; i < n; ++i) {
        views[i] = aq::column_window(*ms[i], c.nb0, c.nb);
        pv[i] = &views[i];
      }
      aq::MatvecFusion f = fu ? *fu : aq::MatvecFusion{};
      f.accumulate = f.accumulate || !first;
      if (f.mode == aq::MatvecFusion::kSwiglu) f.x2 = fu->x2 + c.nb0 * be;
      e = aq::launch_matvec_i8_multi(pv, n, x + c.nb0 * be, ys, s, &f);
      if (e != hipSuccess) break;
      first = false;
    }
  }
  if (prev != m->device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(e, "kernel launch");
  return AQ_OK;
}
}  // namespace

int aq_matvec_multi(const aq_matrix *const *ms, int n, const float *x,
                    float *const *ys, int flags, void *stream) {
  return matvec_multi_impl(ms, n, x, ys, flags, stream, nullptr, "aq_matvec_multi");
}

int aq_matvec_fused(const aq_matrix *const *ms, int n, const float *x,
                    const float *x2, const float *norm_w, float eps,
                    float *const *ys, int flags, void *stream) {
  const int xmodes = flags & (AQ_X_RMSNORM | AQ_X_SWIGLU);
  if (xmodes == (AQ_X_RMSNORM | AQ_X_SWIGLU))
    return fail(AQ_ERR_VALUE, "AQ_X_RMSNORM and AQ_X_SWIGLU exclude each other");
  if ((flags & AQ_X_RMSNORM) && !norm_w) return fail(AQ_ERR_VALUE, "norm_w is NULL");
  if ((flags & AQ_X_SWIGLU) && !x2) return fail(AQ_ERR_VALUE, "x2 is NULL");
  aq::MatvecFusion fu{};
  fu.mode = (flags & AQ_X_RMSNORM) ? aq::MatvecFusion::kNorm
            : (flags & AQ_X_SWIGLU) ? aq::MatvecFusion::kSwiglu
                                    : aq::MatvecFusion::kPlain;
  fu.x2 = x2;
  fu.norm_w = norm_w;
  fu.eps = eps;
  fu.accumulate = (flags & AQ_Y_ACCUMULATE) != 0;
  fu.swiglu_pairs = (flags & AQ_Y_SWIGLU_PAIRS) != 0;
  return matvec_multi_impl(ms, n, x, ys,
                           flags & ~(AQ_X_RMSNORM | AQ_X_SWIGLU | AQ_Y_ACCUMULATE | AQ_Y_SWIGLU_PAIRS),
                           stream, &fu, "aq_matvec_fused");
}

namespace {
// aq_matmul_t, and with ysw (device) the SwiGLU of interleaved (gate, up)
// output pairs into ysw (M x rows/2): formed in the store where the exact
// kernel runs unsplit, else by the pairs kernel over Y.
int matmul_t_impl(const aq_matrix *m, const float *X, int64_t M, float *Y, int precision,
                  int flags, void *stream, float *ysw) {
  if (!m) return fail(AQ_ERR_VALUE, "matrix is NULL");
  if (M < 0) return fail(AQ_ERR_VALUE, "negative batch %lld", (long long)M);
  // AUTO keeps float32 accuracy (qmatrix.py:196-211): a batched prefill
  // through the drop-in stays within the reference's own batched-vs-
  // sequential bar (tests/smoke.py:950-972); bf16 is opt-in.  Small batches
  // run the decode matvec's integer kernel with several x vectors sharing
  // one weight stream (the matvec's accuracy), the others fp32 MFMA: up to
  // 32 rows, and up to 63 for matrices of 2^24 weights or more, where the
  // integer kernel measured faster (Q4_K 14336x4096, M = 63: 260 us against
  // 379 us; 2048x2048, M = 48: 67 us against 49 us).
  const bool big = (double)m->rows * (double)m->cols >= (double)(1 << 24);
  // Formats the exact-integer fp16 kernel takes (aq_matmul_h.hip: weights
  // as exact integers, X in two fp16 pieces, 22 bits per element) run there
  // for FP32, without a split of K so that any M gives the same bits, and
  // for AUTO from 3 rows of X for Q4_K / Q5_K and from 5 for Q6_K and the
  // per-32 block formats, split for speed; AUTO below that runs the integer
  // decode matvec with several x vectors per weight stream (4 per pass up
  // to 4 rows, 8 above).  Measured crossovers (graph-replayed): Q4_K 14336 x
  // 4096 M = 2 13.2 us integer against 17.2 exact, M = 3 20.4 against 17.0;
  // Q8_0 14336 x 4096 M = 4 21.7 against 30.2, M = 5 36.5 against 30.1
  // (Q4_0 33.5 / 28.9, Q5_1 36.6 / 34.7); Q6_K 14336 x 4096 M = 4 24.2
  // against 31.9, M = 5 38.8 against 31.9 (4096 x 14336: 48.6 against 32.2).
  const int64_t exact_min = m->dtype == AQ_Q4_K || m->dtype == AQ_Q5_K ? 3 : 5;
  const bool exact_fp16 = aq::mm_h_supported(m) && (precision == AQ_PREC_FP32 ||
                                                    (precision == AQ_PREC_AUTO && M >= exact_min));
  const bool small = !exact_fp16 && precision == AQ_PREC_AUTO && M <= (big ? 63 : 32) &&
                     !aq::is_dense(m->dtype) && m->rows < INT32_MAX;
  const bool m_invariant = precision == AQ_PREC_FP32;
  if (precision == AQ_PREC_AUTO) precision = AQ_PREC_FP32;
  if (precision != AQ_PREC_FP32 && precision != AQ_PREC_BF16 && precision != AQ_PREC_INT8)
    return fail(AQ_ERR_VALUE, "unknown precision %d", precision);
  if (precision == AQ_PREC_INT8 && m->dtype != AQ_Q8_0)
    return fail(AQ_ERR_VALUE, "int8 matmul_t needs Q8_0 weights (got %s)", dtype_name(m->dtype));
  if (M && ((m->cols && !X) || (m->rows && !Y)))
    return fail(AQ_ERR_VALUE, "X / Y is NULL");
  if (M > ((int64_t)65535 * 128))
    return fail(AQ_ERR_VALUE, "batch %lld too large", (long long)M);
  return run_staged(
      m, X, (size_t)M * m->cols * 4, Y, (size_t)M * m->rows * 4, flags, stream,
      [&](const void *din, void *dout, hipStream_t s) {
        float *yo = static_cast<float *>(dout);
        // the SwiGLU pairs of rows r0 .. r0 + mr of Y
        auto pairs = [&](int64_t r0, int64_t mr) {
          return aq::launch_swiglu(yo + r0 * m->rows, yo + r0 * m->rows + 1, 2,
                                   mr * (m->rows / 2), ysw + r0 * (m->rows / 2), s);
        };
        hipError_t e = hipSuccess;
        if (m->cols == 0) {
          e = fill_zero(yo, M * m->rows, s);
        } else if (exact_fp16) {
          // batches whose X pieces pass 2^31 bytes run in slices of rows
          const int64_t rows_max = std::max<int64_t>(1, ((int64_t)1 << 29) / std::max<int64_t>(1, m->cols));
          for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
            const int64_t mr = std::min(rows_max, M - r0);
            bool fused = false;
            e = aq::launch_matmul_h(m, static_cast<const float *>(din) + r0 * m->cols, mr,
                                    yo + r0 * m->rows, m_invariant, s,
                                    ysw ? ysw + r0 * (m->rows / 2) : nullptr, &fused);
            if (e == hipSuccess && ysw && !fused) e = pairs(r0, mr);
            if (e != hipSuccess) return e;
          }
          return hipSuccess;
        } else if (small) {
          e = aq::launch_matvec_i8_batch(m, static_cast<const float *>(din), M, m->cols, yo,
                                         m->rows, s);
        } else {
          e = aq::launch_matmul_t(m, static_cast<const float *>(din), M, yo, precision, s);
        }
        if (e == hipSuccess && ysw) e = pairs(0, M);
        return e;
      });
}
}  // namespace

int aq_matmul_t(const aq_matrix *m, const float *X, int64_t M, float *Y,
                int precision, int flags, void *stream) {
  return matmul_t_impl(m, X, M, Y, precision, flags, stream, nullptr);
}

int aq_matmul_t_swiglu(const aq_matrix *m, const float *X, int64_t M, float *Z, float *out,
                       int precision, int flags, void *stream) {
  if (!m) return fail(AQ_ERR_VALUE, "matrix is NULL");
  if ((flags & (AQ_IN_DEVICE | AQ_OUT_DEVICE)) != (AQ_IN_DEVICE | AQ_OUT_DEVICE))
    return fail(AQ_ERR_VALUE, "aq_matmul_t_swiglu needs device X, Z and out pointers");
  if (m->rows % 2)
    return fail(AQ_ERR_VALUE, "aq_matmul_t_swiglu needs an even row count (got %lld)",
                (long long)m->rows);
  if (M > 0 && m->rows && (!Z || !out)) return fail(AQ_ERR_VALUE, "Z / out is NULL");
  return matmul_t_impl(m, X, M, Z, precision, flags, stream, out);
}

int aq_dequant_rows(const aq_matrix *m, const int64_t *idx, int64_t n,
                    float *out, int flags, void *stream) {
  if (!m) return fail(AQ_ERR_VALUE, "matrix is NULL");
  if (n < 0) return fail(AQ_ERR_VALUE, "negative row count");
  if (n && (!idx || (m->cols && !out)))
    return fail(AQ_ERR_VALUE, "idx / out is NULL");
  if (!(flags & AQ_IN_DEVICE)) {
    for (int64_t i = 0; i < n; ++i)
      if (idx[i] < 0 || idx[i] >= m->rows)
        return fail(AQ_ERR_INDEX, "row index %lld out of range [0, %lld)",
                    (long long)idx[i], (long long)m->rows);
  } else if (n && m->rows == 0) {
    return fail(AQ_ERR_INDEX, "row gather from an empty matrix");
  }
  // indices go through the input staging slot; the output through slot 1
  return run_staged(
      m, idx, (size_t)n * 8, out, (size_t)n * m->cols * 4, flags, stream,
      [&](const void *din, void *dout, hipStream_t s) {
        return aq::launch_dequant_rows(m, static_cast<const int64_t *>(din), n,
                                       static_cast<float *>(dout), s);
      });
}

// ---- decode step ------------------------------------------------------------

int aq_rmsnorm(const float *x, const float *w, int64_t rows, int64_t n,
               float eps, float *out, void *stream) {
  if (rows < 0 || n < 0) return fail(AQ_ERR_VALUE, "negative shape");
  if (rows && n && (!x || !w || !out)) return fail(AQ_ERR_VALUE, "x / w / out is NULL");
  if (rows > 0x7FFFFFFF) return fail(AQ_ERR_VALUE, "too many rows");
  if (n == 0) return AQ_OK;
  hipError_t e = aq::launch_rmsnorm(x, w, rows, n, eps, out, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? AQ_OK : hip_fail(e, "rmsnorm launch");
}

int aq_add_rmsnorm(float *x, const float *y, const float *w, int64_t rows, int64_t n,
                   float eps, float *out, void *stream) {
  if (rows < 0 || n < 0) return fail(AQ_ERR_VALUE, "negative shape");
  if (rows && n && (!x || !y || !w || !out)) return fail(AQ_ERR_VALUE, "x / y / w / out is NULL");
  if (rows > 0x7FFFFFFF) return fail(AQ_ERR_VALUE, "too many rows");
  if (rows && n && (out == x || out == y)) return fail(AQ_ERR_VALUE, "out aliases x or y");
  hipError_t e = aq::launch_add_rmsnorm(x, y, w, rows, n, eps, out, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? AQ_OK : hip_fail(e, "add_rmsnorm launch");
}

int aq_rope_kv(float *q, const float *k, const float *v, int64_t T, int n_head,
               int n_kv, int head_dim, int n_rot, int neox,
               const float *cos_tab, const float *sin_tab,
               const aq_decode_state *state, int64_t pos0, int64_t n_ctx,
               float *k_cache, float *v_cache, void *stream) {
  if (T < 0 || n_head <= 0 || n_kv <= 0 || head_dim <= 0 || n_ctx <= 0)
    return fail(AQ_ERR_VALUE, "bad rope shape");
  if (head_dim % 2 || n_rot < 0 || n_rot > head_dim || n_rot % 2)
    return fail(AQ_ERR_VALUE, "n_rot %d must be even and <= head_dim %d", n_rot, head_dim);
  if (T && (!q || !k || !v || !k_cache || !v_cache || (n_rot && (!cos_tab || !sin_tab))))
    return fail(AQ_ERR_VALUE, "NULL pointer argument");
  if (!state && (pos0 < 0 || pos0 + T > n_ctx))
    return fail(AQ_ERR_VALUE, "positions %lld..%lld outside the cache of %lld",
                (long long)pos0, (long long)(pos0 + T - 1), (long long)n_ctx);
  if (T * (int64_t)(n_head + n_kv) * (head_dim / 2) > ((int64_t)1 << 40))
    return fail(AQ_ERR_VALUE, "rope batch too large");
  hipError_t e = aq::launch_rope_kv(q, k, v, T, n_head, n_kv, head_dim, n_rot, neox ? 1 : 0,
                                    cos_tab, sin_tab, state, pos0, n_ctx, k_cache,
                                    v_cache, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? AQ_OK : hip_fail(e, "rope launch");
}

int aq_attention_scratch_info(int n_head, int n_kv, int head_dim, int64_t n_ctx,
                              int64_t T, size_t *scratch_bytes, size_t *launch_bytes) {
  if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_ctx <= 0 || T <= 0 || T > 65535)
    return fail(AQ_ERR_VALUE, "bad attention shape");
  if (!aq::attention_supported(head_dim, n_head / n_kv))
    return fail(AQ_ERR_VALUE, "attention supports head_dim 64/128 and groups 1/2/4/8");
  const int G = n_head / n_kv;
  if (scratch_bytes) *scratch_bytes = aq::attention_scratch_bytes(n_kv, head_dim, G, n_ctx, T);
  if (launch_bytes) *launch_bytes = aq::attention_launch_extent_bytes(n_kv, head_dim, G, n_ctx, T);
  return AQ_OK;
}

int aq_attention_batch(const float *q, const float *k_cache, const float *v_cache,
                       int64_t T, int n_head, int n_kv, int head_dim, int64_t n_ctx,
                       const aq_decode_state *state, int64_t pos0, float *out,
                       void *stream) {
  if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_ctx <= 0 || T < 0)
    return fail(AQ_ERR_VALUE, "bad attention shape (n_head %d, n_kv %d)", n_head, n_kv);
  if (!aq::attention_supported(head_dim, n_head / n_kv))
    return fail(AQ_ERR_VALUE, "attention supports head_dim 64/128 and groups 1/2/4/8 "
                "(got head_dim %d, group %d)", head_dim, n_head / n_kv);
  if (T == 0) return AQ_OK;
  if (T > 65535) return fail(AQ_ERR_VALUE, "at most 65535 query tokens per call");
  if (!q || !k_cache || !v_cache || !out) return fail(AQ_ERR_VALUE, "NULL pointer argument");
  if (!state && (pos0 < 0 || pos0 + T > n_ctx))
    return fail(AQ_ERR_VALUE, "positions %lld..%lld outside the cache of %lld",
                (long long)pos0, (long long)(pos0 + T - 1), (long long)n_ctx);
  int dev = 0;
  int rc = current_device(dev);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T > 1 && !getenv("AQ_ATTN_CHUNKED")) {  // the batched (prefill) kernel
    hipError_t e = aq::launch_attention_prefill(q, k_cache, v_cache, n_head, n_kv, head_dim,
                                                n_ctx, state, pos0, T, out, s);
    return e == hipSuccess ? AQ_OK : hip_fail(e, "attention launch");
  }
  const size_t bytes = aq::attention_scratch_bytes(n_kv, head_dim, n_head / n_kv, n_ctx, T);
  float *part = static_cast<float *>(aq::workspace(dev, s, bytes));
  if (!part) return fail(AQ_ERR_RUNTIME, "out of device memory for attention partials");
  hipError_t e = aq::launch_attention(q, k_cache, v_cache, n_head, n_kv, head_dim, n_ctx,
                                      state, pos0, T, part, bytes, out, s);
  return attention_status(e, n_kv, head_dim, n_head / n_kv, n_ctx, T, bytes);
}

int aq_attention(const float *q, const float *k_cache, const float *v_cache,
                 int n_head, int n_kv, int head_dim, int64_t n_ctx,
                 const aq_decode_state *state, int64_t pos0, float *out,
                 void *stream) {
  return aq_attention_batch(q, k_cache, v_cache, 1, n_head, n_kv, head_dim, n_ctx, state,
                            pos0, out, stream);
}

}  // extern "C"

namespace {
int attention_rope_check(int n_head, int n_kv, int head_dim, int n_rot, int neox,
                         const float *q, const float *k, const float *v,
                         const float *cos_tab, const float *sin_tab,
                         const aq_decode_state *state, int64_t pos0, int64_t n_ctx,
                         const float *k_cache, const float *v_cache, const float *out) {
  if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_ctx <= 0)
    return fail(AQ_ERR_VALUE, "bad attention shape (n_head %d, n_kv %d)", n_head, n_kv);
  if (!aq::attention_supported(head_dim, n_head / n_kv))
    return fail(AQ_ERR_VALUE, "attention supports head_dim 64/128 and groups 1/2/4/8 "
                "(got head_dim %d, group %d)", head_dim, n_head / n_kv);
  if (n_rot < 0 || n_rot > head_dim || n_rot % 2 || (neox && n_rot % 8))
    return fail(AQ_ERR_VALUE, "fused rope needs an even n_rot <= head_dim (a multiple "
                "of 8 for neox), got %d", n_rot);
  if (!q || !k || !v || !k_cache || !v_cache || !out || (n_rot && (!cos_tab || !sin_tab)))
    return fail(AQ_ERR_VALUE, "NULL pointer argument");
  if (!state && (pos0 < 0 || pos0 >= n_ctx))
    return fail(AQ_ERR_VALUE, "position %lld outside the cache of %lld", (long long)pos0,
                (long long)n_ctx);
  return AQ_OK;
}

constexpr size_t kNoallocScratchBytes = (size_t)8 << 20;
}  // namespace

// Scratch of aq_attention_rope_noalloc: the decode attention's per-split
// partials (n_head * splits * (head_dim + 4) floats, at most 32 splits) for
// callers that cannot allocate device memory.  Every device the library runs
// on holds one copy for the life of the process.  The array's name is not a
// device address in host code: kernels get the address hipGetSymbolAddress
// returns for the current device, taken once per device (noalloc_scratch).
static __device__ __align__(256) float scratch[kNoallocScratchBytes / sizeof(float)];

namespace {
float *g_scratch_ptr[kMaxDev];
std::mutex g_scratch_mu;

// The scratch address on `device`, which must be the current device.
int noalloc_scratch(int device, float **out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    AQ_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[device] = static_cast<float *>(p);
  }
  *out = g_scratch_ptr[device];
  return AQ_OK;
}
}  // namespace

extern "C" {

int aq_attention_rope_noalloc(float *q, const float *k, const float *v, int n_head,
                              int n_kv, int head_dim, int n_rot, int neox,
                              const float *cos_tab, const float *sin_tab,
                              const aq_decode_state *state, int64_t pos0, int64_t n_ctx,
                              float *k_cache, float *v_cache, float *out, void *stream) {
  int rc = attention_rope_check(n_head, n_kv, head_dim, n_rot, neox, q, k, v, cos_tab,
                                sin_tab, state, pos0, n_ctx, k_cache, v_cache, out);
  if (rc) return rc;
  const size_t bytes = aq::attention_scratch_bytes(n_kv, head_dim, n_head / n_kv, n_ctx, 1);
  if (bytes > kNoallocScratchBytes)
    return fail(AQ_ERR_VALUE,
                "aq_attention_rope_noalloc: the attention partials of %d query heads "
                "(cache of %lld positions) need %zu bytes, more than its %zu-byte static "
                "scratch", n_head, (long long)n_ctx, bytes, kNoallocScratchBytes);
  int dev = 0;
  rc = current_device(dev);
  if (rc) return rc;
  float *part = nullptr;
  rc = noalloc_scratch(dev, &part);
  if (rc) return rc;
  hipError_t e = aq::launch_attention_rope(q, k, v, n_head, n_kv, head_dim, n_rot,
                                           neox ? 1 : 0, cos_tab, sin_tab, n_ctx, state,
                                           pos0, k_cache, v_cache, part, kNoallocScratchBytes,
                                           out, static_cast<hipStream_t>(stream));
  return attention_status(e, n_kv, head_dim, n_head / n_kv, n_ctx, 1, kNoallocScratchBytes);
}

int aq_attention_rope(float *q, const float *k, const float *v, int n_head,
                      int n_kv, int head_dim, int n_rot, int neox,
                      const float *cos_tab, const float *sin_tab,
                      const aq_decode_state *state, int64_t pos0, int64_t n_ctx,
                      float *k_cache, float *v_cache, float *out, void *stream) {
  int rc = attention_rope_check(n_head, n_kv, head_dim, n_rot, neox, q, k, v, cos_tab,
                                sin_tab, state, pos0, n_ctx, k_cache, v_cache, out);
  if (rc) return rc;
  int dev = 0;
  rc = current_device(dev);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t bytes = aq::attention_scratch_bytes(n_kv, head_dim, n_head / n_kv, n_ctx, 1);
  float *part = static_cast<float *>(aq::workspace(dev, s, bytes));
  if (!part) return fail(AQ_ERR_RUNTIME, "out of device memory for attention partials");
  hipError_t e = aq::launch_attention_rope(q, k, v, n_head, n_kv, head_dim, n_rot,
                                           neox ? 1 : 0, cos_tab, sin_tab, n_ctx, state,
                                           pos0, k_cache, v_cache, part, bytes, out, s);
  return attention_status(e, n_kv, head_dim, n_head / n_kv, n_ctx, 1, bytes);
}

int aq_swiglu(const float *gate, const float *up, int64_t n, float *out,
              void *stream) {
  if (n < 0) return fail(AQ_ERR_VALUE, "negative length");
  if (n && (!gate || !up || !out)) return fail(AQ_ERR_VALUE, "NULL pointer argument");
  hipError_t e = aq::launch_swiglu(gate, up, 1, n, out, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? AQ_OK : hip_fail(e, "swiglu launch");
}

int aq_swiglu_pairs(const float *gate_up, int64_t n, float *out, void *stream) {
  if (n < 0) return fail(AQ_ERR_VALUE, "negative length");
  if (n && (!gate_up || !out)) return fail(AQ_ERR_VALUE, "NULL pointer argument");
  hipError_t e = aq::launch_swiglu(gate_up, gate_up + 1, 2, n, out,
                                   static_cast<hipStream_t>(stream));
  return e == hipSuccess ? AQ_OK : hip_fail(e, "swiglu launch");
}

int aq_add_rows(float *x, const float *b, int64_t rows, int64_t n, void *stream) {
  if (rows < 0 || n < 0) return fail(AQ_ERR_VALUE, "negative shape");
  if (rows && n && (!x || !b)) return fail(AQ_ERR_VALUE, "NULL pointer argument");
  hipError_t e = aq::launch_add_rows(x, b, rows, n, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? AQ_OK : hip_fail(e, "add launch");
}

int aq_add(float *x, const float *y, int64_t n, void *stream) {
  if (n < 0) return fail(AQ_ERR_VALUE, "negative length");
  if (n && (!x || !y)) return fail(AQ_ERR_VALUE, "NULL pointer argument");
  hipError_t e = aq::launch_add(x, y, n, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? AQ_OK : hip_fail(e, "add launch");
}

int aq_greedy_advance(const float *logits, int64_t n, aq_decode_state *state,
                      const int64_t *prompt, int64_t n_prompt, int64_t *history,
                      int64_t capacity, int take_argmax, void *stream) {
  if (!state) return fail(AQ_ERR_VALUE, "state is NULL");
  if (take_argmax && (n <= 0 || !logits))
    return fail(AQ_ERR_VALUE, "argmax of an empty sequence");
  if (n > 0xFFFFFFFFll) return fail(AQ_ERR_VALUE, "too many logits");
  if (n_prompt < 0 || (n_prompt && !prompt)) return fail(AQ_ERR_VALUE, "bad prompt");
  if (capacity < 0 || (capacity && !history)) return fail(AQ_ERR_VALUE, "bad history buffer");
  hipError_t e = aq::launch_greedy_advance(logits, n, state, prompt, n_prompt, history,
                                           capacity, take_argmax ? 1 : 0, nullptr, 1, 0, 1.0,
                                           static_cast<hipStream_t>(stream));
  return e == hipSuccess ? AQ_OK : hip_fail(e, "greedy launch");
}

int aq_greedy_advance_penalized(const float *logits, int64_t n, aq_decode_state *state,
                                const int64_t *prompt, int64_t n_prompt, int64_t *history,
                                int64_t capacity, int64_t *window, int64_t last_n,
                                double penalty, int take_argmax, void *stream) {
  if (!state) return fail(AQ_ERR_VALUE, "state is NULL");
  if (take_argmax && (n <= 0 || !logits))
    return fail(AQ_ERR_VALUE, "argmax of an empty sequence");
  if (n > 0xFFFFFFFFll) return fail(AQ_ERR_VALUE, "too many logits");
  if (n_prompt < 0 || (n_prompt && !prompt)) return fail(AQ_ERR_VALUE, "bad prompt");
  if (capacity < 0 || (capacity && !history)) return fail(AQ_ERR_VALUE, "bad history buffer");
  if (!window) return fail(AQ_ERR_VALUE, "window is NULL");
  if (last_n < 1) return fail(AQ_ERR_VALUE, "last_n must be >= 1");
  if (!std::isfinite(penalty))
    return fail(AQ_ERR_VALUE, "penalty must be finite");
  // sample.py:40: a penalty of 0 or 1 leaves the logits as they are
  const int penalize = penalty != 0.0 && penalty != 1.0;
  hipError_t e = aq::launch_greedy_advance(logits, n, state, prompt, n_prompt, history,
                                           capacity, take_argmax ? 1 : 0, window, last_n,
                                           penalize, penalty, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? AQ_OK : hip_fail(e, "greedy launch");
}

}  // extern "C"
