// Calibration: a streaming device copy of known size, the ceiling every bandwidth-bound
// kernel here is measured against and the scale for the HBM byte counters.
//
// The copy reads and writes each 16-byte vector once, with nontemporal loads and stores
// (the policy the fused kernels use for data they touch once). Each thread moves
// `vectors` vectors, 256 threads per workgroup and the workgroup's vectors contiguous:
// thread i of workgroup b handles vectors b * 256 * vectors + i + 256 * j, j < vectors,
// so every wave instruction covers 1 KiB of consecutive memory. All of a thread's loads
// go out before its first store, each from a clamped index with no branch (a load in a
// branch is waited on there); the stores past the end are dropped.
//
// No reference function is replaced: this is measurement infrastructure. A kernel
// moving B bytes (read + write) cannot beat this copy of B / 2 bytes by much, since the
// copy does nothing but move them; the fixed cost of a dispatch (ramp-up until every CU
// has loads in flight, drain of the last waves) is in both.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kCopyBlock = 256;

template <int kVectors>
__global__ __launch_bounds__(kCopyBlock) void stream_copy_kernel(const u32x4* __restrict__ src,
                                                                 u32x4* __restrict__ dst,
                                                                 int64_t vectors) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kCopyBlock * kVectors + threadIdx.x;
  u32x4 held[kVectors];
#pragma unroll
  for (int j = 0; j < kVectors; ++j) {
    const int64_t index = min(first + j * kCopyBlock, vectors - 1);
    held[j] = load_nt(src + index);
  }
  // The loads stay ahead of the stores' branch (see keep_loaded).
#pragma unroll
  for (int j = 0; j < kVectors; ++j) keep_loaded(held[j]);
#pragma unroll
  for (int j = 0; j < kVectors; ++j) {
    const int64_t index = first + j * kCopyBlock;
    if (index < vectors) store_nt(dst + index, held[j]);
  }
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_stream_copy(const void* src, void* dst, int64_t bytes,
                                     int32_t vectors_per_thread, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(bytes >= 0 && bytes % 16 == 0, "stream_copy: bytes must be a multiple of 16");
  OMNIA_REQUIRE(vectors_per_thread == 1 || vectors_per_thread == 2 || vectors_per_thread == 4,
                "stream_copy: vectors_per_thread must be 1, 2 or 4");
  if (bytes == 0) return 0;
  OMNIA_REQUIRE(src && dst && aligned16(src) && aligned16(dst),
                "stream_copy: pointers must be non-null and 16-byte aligned");
  const int64_t vectors = bytes / 16;
  const int64_t per_block = static_cast<int64_t>(kCopyBlock) * vectors_per_thread;
  const int64_t blocks = (vectors + per_block - 1) / per_block;
  OMNIA_REQUIRE(blocks < (int64_t{1} << 31), "stream_copy: too many bytes");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const auto* in = static_cast<const u32x4*>(src);
  auto* out = static_cast<u32x4*>(dst);
  const dim3 grid(static_cast<unsigned>(blocks));
  switch (vectors_per_thread) {
    case 1: stream_copy_kernel<1><<<grid, kCopyBlock, 0, stream>>>(in, out, vectors); break;
    case 2: stream_copy_kernel<2><<<grid, kCopyBlock, 0, stream>>>(in, out, vectors); break;
    default: stream_copy_kernel<4><<<grid, kCopyBlock, 0, stream>>>(in, out, vectors); break;
  }
  return launched("stream_copy");
}
