// aq_calibrate.hip - a streaming-read kernel that measures what one launch can
// read from HBM on this part, the practical ceiling a bandwidth-bound kernel
// of the same byte count is held against (the datasheet peak is not reached
// by any single launch).
//
// Wave w of n reads rows w, w + n, w + 2n, ... of row_bytes each (the decode
// matvec's pattern: one wave per row, rows strided over the waves) through
// buffer resources, `inflight` rows at a time, 16 bytes per lane per load,
// and folds the words into one value so the loads cannot be dropped.  Rows
// past the end have resources of zero bytes: their loads touch no memory.
#include "aq_internal.h"

namespace aq {
namespace {

template <int IF>
__global__ void __launch_bounds__(256)
    k_stream_read(const uint8_t *__restrict__ base, int64_t rows, int row_bytes, int n_waves,
                  unsigned *__restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int w = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int loads = (row_bytes + 1023) / 1024;  // 1 KB (64 lanes x 16 B) per load
  uint32_t acc = 0;
  for (int64_t r = w; r < rows; r += (int64_t)n_waves * IF) {
    uint4 v[IF][4];
#pragma unroll
    for (int i = 0; i < IF; ++i) {
      const int64_t rr = r + (int64_t)i * n_waves;
      const bool live = rr < rows;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t *>(base + (live ? rr : 0) * row_bytes), 0, live ? row_bytes : 0,
          kRsrcWord3);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        v[i][k] = k < loads ? __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                            rs, k * 1024 + lane * 16, 0, 0))
                            : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < IF; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc ^= v[i][k].x ^ v[i][k].y ^ v[i][k].z ^ v[i][k].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;  // practically never: keeps the loads
}

}  // namespace
}  // namespace aq

extern "C" int aq_stream_read(const void *p, int64_t rows, int row_bytes, int waves,
                              int inflight, unsigned *sink, void *stream) {
  if (!p || !sink || rows < 0 || row_bytes <= 0 || row_bytes > 4096 || waves <= 0 ||
      waves % 4)
    return AQ_ERR_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(waves / 4)), block(256);
  const uint8_t *b = static_cast<const uint8_t *>(p);
  switch (inflight) {
    case 1: hipLaunchKernelGGL(aq::k_stream_read<1>, grid, block, 0, s, b, rows, row_bytes, waves, sink); break;
    case 2: hipLaunchKernelGGL(aq::k_stream_read<2>, grid, block, 0, s, b, rows, row_bytes, waves, sink); break;
    case 4: hipLaunchKernelGGL(aq::k_stream_read<4>, grid, block, 0, s, b, rows, row_bytes, waves, sink); break;
    default: return AQ_ERR_VALUE;
  }
  return hipGetLastError() == hipSuccess ? AQ_OK : AQ_ERR_RUNTIME;
}
