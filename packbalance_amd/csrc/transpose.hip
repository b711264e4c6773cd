// Batched matrix transpose for gfx950: dst[b][c][r] = src[b][r][c].
//
// Builds the transposed compute-dtype weight copies that the input-gradient
// GEMMs read (dx = dy W runs fastest in hipBLASLt with W stored [K, N]): one
// launch transposes one weight kind of every layer, the layers sitting at a
// constant stride in the flat parameter store.  Pure data movement, bound by
// HBM: each element is read once and written once (2 x elem bytes).
//
// One workgroup per 64 x 64 tile of one matrix.  Full tiles with 16-byte
// aligned rows move 16-byte vectors both ways (rows of the source tile in,
// rows of the destination tile out) through an LDS tile padded by two
// elements per row; edge tiles and unaligned shapes go element by element
// with bounds checks.
#include "common.hpp"

namespace pb {
namespace {

constexpr int kTile = 64;
constexpr int kThreads = 256;

template <typename T>  // element bits: uint16_t (bf16/fp16) or uint32_t (fp32)
__global__ __launch_bounds__(kThreads) void transpose_tiles(const T *__restrict__ src,
                                                            int64_t src_bs, int64_t src_rs,
                                                            T *__restrict__ dst, int rows,
                                                            int cols, int vec) {
  __shared__ T t[kTile][kTile + 2];
  const int r0 = blockIdx.y * kTile, c0 = blockIdx.x * kTile;
  const T *s = src + (int64_t)blockIdx.z * src_bs;
  T *d = dst + (int64_t)blockIdx.z * rows * cols;
  constexpr int V = 16 / sizeof(T);  // elements per 16-byte vector
  constexpr int CH = kTile / V;      // vectors per tile row
  if (vec && r0 + kTile <= rows && c0 + kTile <= cols) {
    for (int k = threadIdx.x; k < kTile * CH; k += kThreads) {
      const int r = k / CH, ch = k % CH;
      const u32x4 raw =
          __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(s + (int64_t)(r0 + r) * src_rs + c0 + ch * V));
      const T *e = reinterpret_cast<const T *>(&raw);
#pragma unroll
      for (int i = 0; i < V; ++i) t[r][ch * V + i] = e[i];
    }
    __syncthreads();
    for (int k = threadIdx.x; k < kTile * CH; k += kThreads) {
      const int c = k / CH, ch = k % CH;
      u32x4 raw;
      T *e = reinterpret_cast<T *>(&raw);
#pragma unroll
      for (int i = 0; i < V; ++i) e[i] = t[ch * V + i][c];
      *reinterpret_cast<u32x4 *>(d + (int64_t)(c0 + c) * rows + r0 + ch * V) = raw;
    }
  } else {
    for (int k = threadIdx.x; k < kTile * kTile; k += kThreads) {
      const int r = k / kTile, c = k % kTile;
      if (r0 + r < rows && c0 + c < cols) t[r][c] = s[(int64_t)(r0 + r) * src_rs + c0 + c];
    }
    __syncthreads();
    for (int k = threadIdx.x; k < kTile * kTile; k += kThreads) {
      const int c = k / kTile, r = k % kTile;
      if (r0 + r < rows && c0 + c < cols) d[(int64_t)(c0 + c) * rows + r0 + r] = t[r][c];
    }
  }
}

}  // namespace
}  // namespace pb

extern "C" int pb_transpose_batched(const void *src, int64_t src_batch_stride,
                                    int64_t src_row_stride, void *dst, int64_t batch,
                                    int64_t rows, int64_t cols, int elem_bytes, void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(elem_bytes == 2 || elem_bytes == 4, "pb_transpose_batched: elements must be 2 or 4 bytes");
  PB_CHECK_ARG(batch >= 0 && rows >= 0 && cols >= 0 && src_row_stride >= cols &&
                   (batch <= 1 || src_batch_stride >= rows * src_row_stride),
               "pb_transpose_batched: bad sizes or strides");
  if (batch == 0 || rows == 0 || cols == 0) return PB_OK;
  PB_CHECK_ARG(src && dst, "pb_transpose_batched: null argument");
  PB_CHECK_SUPPORTED(rows < (int64_t)kTile * 65535 && cols < (int64_t)1 << 31 && batch <= 65535 &&
                         rows * cols < (int64_t)1 << 31,
                     "pb_transpose_batched: a matrix of at most 2^31 elements, %d batches",
                     65535);
  const int64_t eb = elem_bytes;
  const int vec = reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(dst) % 16 == 0 && (src_row_stride * eb) % 16 == 0 &&
                  (src_batch_stride * eb) % 16 == 0 && (rows * eb) % 16 == 0;
  dim3 grid((unsigned)((cols + kTile - 1) / kTile), (unsigned)((rows + kTile - 1) / kTile),
            (unsigned)batch);
  if (elem_bytes == 2)
    hipLaunchKernelGGL(transpose_tiles<uint16_t>, grid, dim3(kThreads), 0, as_stream(stream),
                       static_cast<const uint16_t *>(src), src_batch_stride, src_row_stride,
                       static_cast<uint16_t *>(dst), (int)rows, (int)cols, vec);
  else
    hipLaunchKernelGGL(transpose_tiles<uint32_t>, grid, dim3(kThreads), 0, as_stream(stream),
                       static_cast<const uint32_t *>(src), src_batch_stride, src_row_stride,
                       static_cast<uint32_t *>(dst), (int)rows, (int)cols, vec);
  return launch_status("pb_transpose_batched");
}
