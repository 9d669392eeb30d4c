// Diagnostic read kernels: the HBM read rate the paged decode's access pattern
// can reach on this device, measured with the same clocks and settling as the
// decode itself.  No reference counterpart (the reference has no bandwidth
// ceiling to compare against); bench.py times them as "ceiling" legs.
//
//   paged_gather_kernel  reads every (page, kv head) K block and V block that a
//                        paged decode over the same CSR page table reads (whole
//                        pages, `page_size` x `head_dim` fp16 each), blocks
//                        dealt round-robin to waves, two blocks in flight per
//                        wave, and nothing else: no scores, no softmax, no
//                        merges.
//   stream_read_kernel   reads one contiguous range linearly, four 16-byte loads
//                        in flight per thread.
//
// Both XOR what they read into a register and store it only in the (never
// matching) case that it equals a caller-given key, so the loads cannot be
// removed and nothing else is written.
#include "akt_common.hpp"
#include "akt_host.hpp"

namespace akt {
namespace {

constexpr int kDiagThreads = 256;

// NL = 1 KB rows of 64 lanes x 16 bytes per K (and per V) block.
template <int NL>
__global__ __launch_bounds__(kDiagThreads) void paged_gather_kernel(
    const char* __restrict__ pool, const int32_t* __restrict__ indices, int64_t total_pages,
    int64_t num_kv_heads, int64_t num_pool_pages, int64_t page_bytes, int64_t head_bytes,
    int64_t v_bytes, uint32_t key, uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (kDiagThreads / 64) + (threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * (kDiagThreads / 64);
  const int64_t nblk = total_pages * num_kv_heads;
  uint4_t acc = {0, 0, 0, 0};
  uint4_t buf[2][2 * NL];
  // Block b: kv head b / total_pages, CSR position b % total_pages (kv-head
  // major, as a decode unit walks one kv head's pages).  Blocks past the end
  // and invalid page ids read the pool's first block instead (always mapped).
  auto issue = [&](int64_t b, uint4_t (&d)[2 * NL]) {
    int64_t off = 0;
    if (b < nblk) {
      const int64_t h = b / total_pages;
      const int32_t page = indices[b - h * total_pages];
      if (page >= 0 && page < num_pool_pages) off = (int64_t)page * page_bytes + h * head_bytes;
    }
    const char* kp = pool + off + lane * 16;
#pragma unroll
    for (int j = 0; j < NL; ++j) d[j] = ld16(kp + j * 1024);
#pragma unroll
    for (int j = 0; j < NL; ++j) d[NL + j] = ld16(kp + v_bytes + j * 1024);
  };
  issue(wave, buf[0]);
  issue(wave + nw, buf[1]);
  for (int64_t b = wave; b < nblk; b += 2 * nw) {
#pragma unroll
    for (int j = 0; j < 2 * NL; ++j) acc ^= buf[0][j];
    issue(b + 2 * nw, buf[0]);
    if (b + nw < nblk) {
#pragma unroll
      for (int j = 0; j < 2 * NL; ++j) acc ^= buf[1][j];
    }
    issue(b + 3 * nw, buf[1]);
  }
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == key) sink[0] = x;
}

__global__ __launch_bounds__(kDiagThreads) void stream_read_kernel(const uint4_t* __restrict__ p,
                                                                   int64_t n, uint32_t key,
                                                                   uint32_t* sink) {
  uint4_t acc = {0, 0, 0, 0};
  const int64_t stride = (int64_t)gridDim.x * kDiagThreads;
  int64_t i = (int64_t)blockIdx.x * kDiagThreads + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const uint4_t a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n; i += stride) acc ^= p[i];
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == key) sink[0] = x;
}

// Workgroups of the diagnostic launches: two per CU for the gather (the paged
// decode's occupancy), four per CU for the linear read (its best grid here).
constexpr unsigned kGatherGrid = 512;
constexpr unsigned kStreamGrid = 1024;

}  // namespace
}  // namespace akt

using namespace akt;

extern "C" int akt_diag_paged_gather(const void* kv_cache, const int32_t* kv_page_indices,
                                     int64_t total_pages, int64_t num_kv_heads,
                                     int64_t head_dim, int64_t page_size, int64_t num_pool_pages,
                                     const int64_t kv_stride[5], uint32_t* sink, void* stream) {
  clear_error();
  AKT_CHECK(total_pages >= 0 && num_kv_heads > 0 && head_dim > 0 && page_size > 0 &&
                num_pool_pages >= 0,
            "sizes must be positive");
  AKT_CHECK(kv_stride && kv_stride[4] == 1 && kv_stride[3] == head_dim,
            "each (page, kv head) block must be contiguous");
  AKT_CHECK(kv_stride[0] >= 0 && kv_stride[1] >= 0 && kv_stride[2] >= 0, "strides must be >= 0");
  AKT_CHECK(aligned16(kv_cache) && (kv_stride[0] * 2) % 16 == 0 && (kv_stride[1] * 2) % 16 == 0 &&
                (kv_stride[2] * 2) % 16 == 0,
            "blocks must be 16-byte aligned");
  AKT_CHECK(sink != nullptr, "sink is required");
  if (total_pages == 0 || num_pool_pages == 0) return AKT_OK;
  const int64_t block = page_size * head_dim * 2;
  const int NL = (int)(block / 1024);
  if (block % 1024 != 0 || (NL != 2 && NL != 4 && NL != 8 && NL != 16))
    return set_error(AKT_ERR_UNSUPPORTED,
                     "paged gather reads blocks of 2, 4, 8 or 16 KB (page_size * head_dim * 2 = "
                     "%lld bytes)",
                     (long long)block);
  const char* pool = (const char*)kv_cache;
  const int64_t pb = kv_stride[0] * 2, hb = kv_stride[2] * 2, vb = kv_stride[1] * 2;
  hipStream_t st = (hipStream_t)stream;
  const uint32_t key = 0x9e3779b9u;
  KernelTimer timer;
  switch (NL) {
    case 2: timer.launch(paged_gather_kernel<2>, dim3(kGatherGrid), dim3(kDiagThreads), 0, st, pool, kv_page_indices, total_pages, num_kv_heads, num_pool_pages, pb, hb, vb, key, sink); break;
    case 4: timer.launch(paged_gather_kernel<4>, dim3(kGatherGrid), dim3(kDiagThreads), 0, st, pool, kv_page_indices, total_pages, num_kv_heads, num_pool_pages, pb, hb, vb, key, sink); break;
    case 8: timer.launch(paged_gather_kernel<8>, dim3(kGatherGrid), dim3(kDiagThreads), 0, st, pool, kv_page_indices, total_pages, num_kv_heads, num_pool_pages, pb, hb, vb, key, sink); break;
    default: timer.launch(paged_gather_kernel<16>, dim3(kGatherGrid), dim3(kDiagThreads), 0, st, pool, kv_page_indices, total_pages, num_kv_heads, num_pool_pages, pb, hb, vb, key, sink); break;
  }
  return check_launch("paged_gather_kernel");
}

extern "C" int akt_diag_stream_read(const void* data, int64_t bytes, uint32_t* sink,
                                    void* stream) {
  clear_error();
  AKT_CHECK(bytes >= 0 && bytes % 16 == 0, "bytes must be a non-negative multiple of 16");
  AKT_CHECK(aligned16(data) && sink != nullptr, "data must be 16-byte aligned; sink is required");
  if (bytes == 0) return AKT_OK;
  KernelTimer timer;
  timer.launch(stream_read_kernel, dim3(kStreamGrid), dim3(kDiagThreads), 0, (hipStream_t)stream,
               (const uint4_t*)data, bytes / 16, 0x9e3779b9u, sink);
  return check_launch("stream_read_kernel");
}
