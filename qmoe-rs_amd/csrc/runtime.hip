// runtime.hip -- library plumbing: error strings, device info, HBM buffers,
// streams and two small utility kernels (f32 -> bf16, normal fill).
//
// The buffer API is the device-side replacement of the host storage in
// src/tensor.rs:1-122: the engine owns HBM allocations and hands their
// addresses to the attention entry points.

#include <cmath>
#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "internal.hpp"

namespace qmla {

namespace {
thread_local std::string t_err;
}

void set_error_msg(const char *fmt, ...) {
  char buf[768];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_err = buf;
}
const char *error_msg() { return t_err.c_str(); }
void clear_error() { t_err.clear(); }

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cached;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cached.size() <= dev) cached.resize(dev + 1, 0);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    cached[dev] = n;
  }
  return cached[dev];
}

qmla_status ensure_dynamic_lds(const void *fn, size_t bytes) {
  static std::mutex mu;
  static std::map<std::pair<const void *, int>, size_t> done;
  int dev = 0;
  QMLA_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  size_t &have = done[{fn, dev}];
  if (have >= bytes) return QMLA_OK;
  QMLA_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
  have = bytes;
  return QMLA_OK;
}

// ------------------------------------------------------------- kernels ----

__global__ void k_f32_to_bf16(const float *__restrict__ src, uint16_t *__restrict__ dst,
                              size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = f32_to_bf16_bits(src[i]);
}

__device__ inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

// Counter-based normal generator (SplitMix64 outputs 2i, 2i+1 -> Box-Muller
// in f32).  Deterministic per (seed, i); used for synthetic benchmark data.
__global__ void k_fill_normal(float *__restrict__ dst, size_t n, uint64_t seed, float mean,
                              float sd) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    uint64_t a = mix64(seed + (2 * i + 1) * 0x9E3779B97F4A7C15ULL);
    uint64_t b = mix64(seed + (2 * i + 2) * 0x9E3779B97F4A7C15ULL);
    float u1 = ((float)(a >> 40) + 1.0f) * (1.0f / 16777216.0f);
    float u2 = (float)(b >> 40) * (1.0f / 16777216.0f);
    float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853071795864f * u2);
    dst[i] = mean + sd * z;
  }
}

// Zero fill of n bytes at p: the bytes before the first 16-byte boundary
// and after the last one go one by one, the aligned middle as 16-byte
// stores, grid-stride.
__global__ void k_zero_bytes(uint8_t *__restrict__ p, size_t n) {
  const size_t head = std::min<size_t>(n, (16 - ((uintptr_t)p & 15)) & 15);
  const size_t nvec = (n - head) / 16;
  const size_t tail0 = head + nvec * 16;
  const size_t i0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  uint4 *body = reinterpret_cast<uint4 *>(p + head);
  for (size_t i = i0; i < nvec; i += stride) body[i] = make_uint4(0, 0, 0, 0);
  if (i0 < head) p[i0] = 0;
  if (i0 < n - tail0) p[tail0 + i0] = 0;
}

qmla_status zero_bytes(void *dst, size_t bytes, hipStream_t s) {
  if (bytes == 0) return QMLA_OK;
  const size_t nvec = bytes / 16 + 1;
  const unsigned blocks = (unsigned)std::min<size_t>((nvec + 255) / 256, 4096);
  k_zero_bytes<<<dim3(blocks), dim3(256), 0, s>>>(static_cast<uint8_t *>(dst), bytes);
  QMLA_LAUNCH_CHECK("k_zero_bytes");
  return QMLA_OK;
}

}  // namespace qmla

using namespace qmla;

extern "C" {

int qmla_version(void) { return QMLA_VERSION; }

const char *qmla_last_error(void) { return error_msg(); }

const char *qmla_status_string(qmla_status s) {
  switch (s) {
    case QMLA_OK: return "QMLA_OK";
    case QMLA_ERR_INVALID_ARG: return "QMLA_ERR_INVALID_ARG";
    case QMLA_ERR_SHAPE: return "QMLA_ERR_SHAPE";
    case QMLA_ERR_UNSUPPORTED: return "QMLA_ERR_UNSUPPORTED";
    case QMLA_ERR_HIP: return "QMLA_ERR_HIP";
    case QMLA_ERR_OOM: return "QMLA_ERR_OOM";
    case QMLA_ERR_CAPACITY: return "QMLA_ERR_CAPACITY";
    case QMLA_ERR_WORKSPACE: return "QMLA_ERR_WORKSPACE";
  }
  return "QMLA_ERR_UNKNOWN";
}

qmla_status qmla_device_info(int *device, int *cu_count, char *arch_name, size_t arch_len) {
  int dev = 0;
  QMLA_HIP(hipGetDevice(&dev));
  if (device) *device = dev;
  if (cu_count) *cu_count = device_cu_count();
  if (arch_name && arch_len > 0) {
    hipDeviceProp_t p;
    QMLA_HIP(hipGetDeviceProperties(&p, dev));
    std::strncpy(arch_name, p.gcnArchName, arch_len - 1);
    arch_name[arch_len - 1] = 0;
  }
  return QMLA_OK;
}

qmla_status qmla_buffer_alloc(size_t bytes, void **out) {
  QMLA_REQUIRE(out != nullptr, QMLA_ERR_INVALID_ARG, "out is NULL");
  QMLA_REQUIRE(bytes > 0, QMLA_ERR_INVALID_ARG, "bytes must be > 0");
  *out = nullptr;
  QMLA_HIP(hipMalloc(out, bytes));
  return QMLA_OK;
}

qmla_status qmla_buffer_free(void *ptr) {
  if (ptr) QMLA_HIP(hipFree(ptr));
  return QMLA_OK;
}

qmla_status qmla_memcpy_h2d(void *dst, const void *src, size_t bytes, qmla_stream stream) {
  QMLA_REQUIRE(dst && src, QMLA_ERR_INVALID_ARG, "NULL pointer");
  if (bytes) QMLA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
  return QMLA_OK;
}

qmla_status qmla_memcpy_d2h(void *dst, const void *src, size_t bytes, qmla_stream stream) {
  QMLA_REQUIRE(dst && src, QMLA_ERR_INVALID_ARG, "NULL pointer");
  if (bytes) QMLA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
  return QMLA_OK;
}

qmla_status qmla_memcpy_d2d(void *dst, const void *src, size_t bytes, qmla_stream stream) {
  QMLA_REQUIRE(dst && src, QMLA_ERR_INVALID_ARG, "NULL pointer");
  if (bytes)
    QMLA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
  return QMLA_OK;
}

qmla_status qmla_memset_zero(void *dst, size_t bytes, qmla_stream stream) {
  QMLA_REQUIRE(dst, QMLA_ERR_INVALID_ARG, "NULL pointer");
  return zero_bytes(dst, bytes, as_stream(stream));
}

qmla_status qmla_stream_create(qmla_stream *out) {
  QMLA_REQUIRE(out, QMLA_ERR_INVALID_ARG, "out is NULL");
  hipStream_t s = nullptr;
  QMLA_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = reinterpret_cast<qmla_stream>(s);
  return QMLA_OK;
}

qmla_status qmla_stream_destroy(qmla_stream stream) {
  if (stream) QMLA_HIP(hipStreamDestroy(as_stream(stream)));
  return QMLA_OK;
}

qmla_status qmla_stream_synchronize(qmla_stream stream) {
  QMLA_HIP(hipStreamSynchronize(as_stream(stream)));
  return QMLA_OK;
}

qmla_status qmla_f32_to_bf16(const float *src, uint16_t *dst, size_t n, qmla_stream stream) {
  QMLA_REQUIRE(src && dst, QMLA_ERR_INVALID_ARG, "NULL pointer");
  if (n == 0) return QMLA_OK;
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  k_f32_to_bf16<<<dim3((unsigned)blocks), dim3(256), 0, as_stream(stream)>>>(src, dst, n);
  QMLA_LAUNCH_CHECK("k_f32_to_bf16");
  return QMLA_OK;
}

qmla_status qmla_fill_normal_f32(float *dst, size_t n, uint64_t seed, float mean, float std_,
                                 qmla_stream stream) {
  QMLA_REQUIRE(dst, QMLA_ERR_INVALID_ARG, "NULL pointer");
  if (n == 0) return QMLA_OK;
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  k_fill_normal<<<dim3((unsigned)blocks), dim3(256), 0, as_stream(stream)>>>(dst, n, seed, mean,
                                                                            std_);
  QMLA_LAUNCH_CHECK("k_fill_normal");
  return QMLA_OK;
}

}  // extern "C"
