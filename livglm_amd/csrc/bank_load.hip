// Checkpoint shards -> HBM expert bank.
//
// The reference refills a bounded slot cache from SSD per routed expert
// (native_expert_ssd.py:318-339 opens one direct reader per shard,
// native_expert_ssd.py:367-387 copies one expert's tensors into its slot).  A
// whole layer's experts fit in HBM here, so loading is a one-time bulk move:
// worker threads pread each expert's byte range (one contiguous record of six
// U8 tensors, expert_source.py:249-276) into pinned host staging, one DMA per
// staging chunk moves it to device memory, and a scatter kernel moves every
// tensor of every record to its slot in the stacked bank tensors.
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "glm_common.h"

namespace glm {

constexpr long long kReadPiece = 2ll << 20;  // one pread call at most
constexpr int kScatterThreads = 256;
constexpr long long kScatterBlockBytes = 64ll << 10;  // bytes per workgroup
constexpr int kMaxSegmentsPerLaunch = 65535;          // grid.y

// Segment table row: {source offset in the staging buffer, destination
// address, bytes}.  One workgroup copies kScatterBlockBytes of one segment:
// 16-byte vector copies when source and destination are both 16-byte
// aligned, byte copies otherwise.
__global__ __launch_bounds__(kScatterThreads) void bank_scatter_kernel(const uint8_t *staging,
                                                                       const int64_t *segments) {
  const int64_t *row = segments + 3ll * blockIdx.y;
  const long long src_off = row[0];
  uint8_t *dst = reinterpret_cast<uint8_t *>(row[1]);
  const long long bytes = row[2];
  const long long begin = (long long)blockIdx.x * kScatterBlockBytes;
  if (begin >= bytes) return;
  const long long end = begin + kScatterBlockBytes < bytes ? begin + kScatterBlockBytes : bytes;
  const uint8_t *src = staging + src_off;
  long long tail = begin;
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0) {
    const long long vend = begin + ((end - begin) & ~15ll);
    for (long long i = begin + 16ll * threadIdx.x; i < vend; i += 16ll * kScatterThreads)
      *reinterpret_cast<glm_u32x4 *>(dst + i) = *reinterpret_cast<const glm_u32x4 *>(src + i);
    tail = vend;
  }
  for (long long i = tail + threadIdx.x; i < end; i += kScatterThreads) dst[i] = src[i];
}

}  // namespace glm

using namespace glm;

extern "C" int glm_file_read_ranges(const char *path, int n, const int64_t *offset,
                                    const int64_t *length, void *const *dst, int threads,
                                    int flags) {
  glm::clear_error();
  GLM_REQUIRE(path != nullptr, GLM_ERR_INVALID_ARGUMENT, "file_read_ranges: null path");
  GLM_REQUIRE(n >= 0, GLM_ERR_INVALID_ARGUMENT, "file_read_ranges: negative range count");
  GLM_REQUIRE(n == 0 || (offset && length && dst), GLM_ERR_INVALID_ARGUMENT,
              "file_read_ranges: null range table");
  GLM_REQUIRE(threads >= 1 && threads <= 256, GLM_ERR_INVALID_ARGUMENT,
              "file_read_ranges: threads must be in 1..256, got %d", threads);
  GLM_REQUIRE((flags & ~GLM_READ_DROP_CACHE) == 0, GLM_ERR_INVALID_ARGUMENT,
              "file_read_ranges: unknown flags %d", flags);
  for (int i = 0; i < n; ++i) {
    GLM_REQUIRE(offset[i] >= 0 && length[i] >= 0, GLM_ERR_INVALID_ARGUMENT,
                "file_read_ranges: range %d has offset %lld length %lld", i,
                (long long)offset[i], (long long)length[i]);
    GLM_REQUIRE(length[i] == 0 || dst[i] != nullptr, GLM_ERR_INVALID_ARGUMENT,
                "file_read_ranges: range %d has no destination", i);
  }
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  GLM_REQUIRE(fd >= 0, GLM_ERR_INVALID_ARGUMENT, "file_read_ranges: cannot open %s: %s", path,
              strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    const int err = errno;
    close(fd);
    GLM_REQUIRE(false, GLM_ERR_INVALID_ARGUMENT, "file_read_ranges: cannot stat %s: %s", path,
                strerror(err));
  }
  struct Piece {
    long long off, len;
    uint8_t *dst;
  };
  std::vector<Piece> pieces;
  for (int i = 0; i < n; ++i) {
    if (offset[i] + length[i] > (long long)st.st_size) {
      close(fd);
      GLM_REQUIRE(false, GLM_ERR_INVALID_ARGUMENT,
                  "file_read_ranges: range %d [%lld, %lld) is beyond the end of %s (%lld bytes)",
                  i, (long long)offset[i], (long long)(offset[i] + length[i]), path,
                  (long long)st.st_size);
    }
    for (long long p = 0; p < length[i]; p += kReadPiece)
      pieces.push_back({offset[i] + p, std::min<long long>(kReadPiece, length[i] - p),
                        static_cast<uint8_t *>(dst[i]) + p});
  }
  std::atomic<size_t> next{0};
  std::mutex mu;
  std::string failure;
  auto worker = [&]() {
    for (;;) {
      const size_t j = next.fetch_add(1);
      if (j >= pieces.size()) return;
      const Piece &pc = pieces[j];
      long long done = 0;
      while (done < pc.len) {
        const ssize_t got = pread(fd, pc.dst + done, (size_t)(pc.len - done), pc.off + done);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) {
          std::lock_guard<std::mutex> lock(mu);
          if (failure.empty())
            failure = std::string("pread at ") + std::to_string(pc.off + done) + " of " + path +
                      ": " + (got < 0 ? strerror(errno) : "unexpected end of file");
          next.store(pieces.size());  // the other workers stop after their piece
          return;
        }
        done += got;
      }
    }
  };
  const int nthreads = (int)std::min<size_t>((size_t)threads, std::max<size_t>(1, pieces.size()));
  std::vector<std::thread> pool;
  pool.reserve(nthreads > 1 ? nthreads - 1 : 0);
  for (int t = 1; t < nthreads; ++t) pool.emplace_back(worker);
  worker();
  for (auto &th : pool) th.join();
  if (failure.empty() && (flags & GLM_READ_DROP_CACHE))
    for (int i = 0; i < n; ++i) posix_fadvise(fd, offset[i], length[i], POSIX_FADV_DONTNEED);
  close(fd);
  GLM_REQUIRE(failure.empty(), GLM_ERR_INVALID_ARGUMENT, "file_read_ranges: %s",
              failure.c_str());
  return GLM_OK;
}

extern "C" int glm_bank_scatter(void *stream, const uint8_t *staging, int64_t staging_bytes,
                                const int64_t *segments, int n, int64_t *device_table) {
  glm::clear_error();
  GLM_REQUIRE(n >= 0 && staging_bytes >= 0, GLM_ERR_INVALID_ARGUMENT,
              "bank_scatter: negative segment count or staging size");
  if (n == 0) return GLM_OK;
  GLM_REQUIRE(staging && segments && device_table, GLM_ERR_INVALID_ARGUMENT,
              "bank_scatter: null pointer");
  long long max_bytes = 0;
  for (int i = 0; i < n; ++i) {
    const int64_t *row = segments + 3ll * i;
    GLM_REQUIRE(row[0] >= 0 && row[2] >= 0 && row[0] + row[2] <= staging_bytes,
                GLM_ERR_INVALID_ARGUMENT,
                "bank_scatter: segment %d [%lld, +%lld) is outside the %lld-byte staging buffer", i,
                (long long)row[0], (long long)row[2], (long long)staging_bytes);
    GLM_REQUIRE(row[2] == 0 || row[1] != 0, GLM_ERR_INVALID_ARGUMENT,
                "bank_scatter: segment %d has no destination", i);
    max_bytes = std::max<long long>(max_bytes, row[2]);
  }
  if (max_bytes == 0) return GLM_OK;
  const long long blocks = (max_bytes + kScatterBlockBytes - 1) / kScatterBlockBytes;
  GLM_REQUIRE(blocks <= 0x7fffffffll, GLM_ERR_UNSUPPORTED_SHAPE, "bank_scatter: segment too large");
  GLM_HIP_CHECK(hipMemcpyAsync(device_table, segments, (size_t)n * 3 * sizeof(int64_t),
                               hipMemcpyHostToDevice, (hipStream_t)stream));
  for (int first = 0; first < n; first += kMaxSegmentsPerLaunch) {
    const int count = std::min(kMaxSegmentsPerLaunch, n - first);
    hipLaunchKernelGGL(bank_scatter_kernel, dim3((unsigned)blocks, (unsigned)count),
                       dim3(kScatterThreads), 0, (hipStream_t)stream, staging,
                       device_table + 3ll * first);
    GLM_LAUNCH_CHECK("bank_scatter_kernel");
  }
  return GLM_OK;
}
