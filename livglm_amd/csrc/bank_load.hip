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

constexpr int kScatterCols = 4;

// Segment table row: {source offset in the staging buffer, destination
// address, bytes, tile_k}.  One workgroup copies kScatterBlockBytes of one
// segment: tile_k > 0 marks a whole MXFP4 matrix with tile_k codes a row,
// written tile-major in 16-byte pieces (the destination aligned, the source
// wherever the checkpoint put it); otherwise 16-byte vector copies when
// source and destination are both 16-byte aligned, byte copies else.
__global__ __launch_bounds__(kScatterThreads) void bank_scatter_kernel(const uint8_t *staging,
                                                                       const int64_t *segments) {
  const int64_t *row = segments + (long long)kScatterCols * blockIdx.y;
  const long long src_off = row[0];
  uint8_t *dst = reinterpret_cast<uint8_t *>(row[1]);
  const long long bytes = row[2];
  const long long tile_k = row[3];
  const long long begin = (long long)blockIdx.x * kScatterBlockBytes;
  if (begin >= bytes) return;
  const long long end = begin + kScatterBlockBytes < bytes ? begin + kScatterBlockBytes : bytes;
  const uint8_t *src = staging + src_off;
  if (tile_k > 0) {
    const long long ppr = tile_k / 32;  // 16-byte pieces a row
    const bool aligned = (reinterpret_cast<uintptr_t>(src) & 15u) == 0;
    for (long long i = begin + 16ll * threadIdx.x; i < end; i += 16ll * kScatterThreads) {
      const long long piece = i >> 4;
      uint8_t *d = dst + 16 * mxfp4_tile_piece(piece / ppr, piece % ppr, tile_k);
      if (aligned) {
        *reinterpret_cast<glm_u32x4 *>(d) = *reinterpret_cast<const glm_u32x4 *>(src + i);
      } else {
#pragma unroll
        for (int b = 0; b < 16; ++b) d[b] = src[i + b];
      }
    }
    return;
  }
  long long tail = begin;
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0) {
    const long long vend = begin + ((end - begin) & ~15ll);
    for (long long i = begin + 16ll * threadIdx.x; i < vend; i += 16ll * kScatterThreads)
      *reinterpret_cast<glm_u32x4 *>(dst + i) = *reinterpret_cast<const glm_u32x4 *>(src + i);
    tail = vend;
  }
  for (long long i = tail + threadIdx.x; i < end; i += kScatterThreads) dst[i] = src[i];
}

// count row-major MXFP4 matrices of per_matrix 16-byte pieces -> tile-major
// (grid-stride over the source pieces; reads coalesced, writes whole pieces).
__global__ __launch_bounds__(kScatterThreads) void mxfp4_tile_kernel(const uint8_t *src,
                                                                     uint8_t *dst, long long pieces,
                                                                     long long per_matrix, int K) {
  const long long ppr = K / 32;
  for (long long i = (long long)blockIdx.x * kScatterThreads + threadIdx.x; i < pieces;
       i += (long long)gridDim.x * kScatterThreads) {
    const long long m = i / per_matrix, rem = i - m * per_matrix;
    const long long o = m * per_matrix + mxfp4_tile_piece(rem / ppr, rem % ppr, K);
    *reinterpret_cast<glm_u32x4 *>(dst + 16 * o) =
        *reinterpret_cast<const glm_u32x4 *>(src + 16 * i);
  }
}

// ScaleX Mode-A records (scale_codec.py:35-91) decoded into raw E8M0 bytes.
// Table row (13 x int64): staging offset of the record, encoded bytes, raw
// bytes, codec (0 raw, 1 one bit, 2 two bits), the four palette bytes packed
// little-endian, primary bytes, exception count, then three (destination,
// bytes) pairs that receive the raw bytes in order (gate, down, up scales).
constexpr int kScalexCols = 13;
constexpr int kScalexHeader = 24;
constexpr int kScalexBlock = 4096;  // scales per workgroup

__device__ __forceinline__ uint32_t load_u32_le(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

__global__ __launch_bounds__(kScatterThreads) void scalex_decode_kernel(const uint8_t *staging,
                                                                        const int64_t *table) {
  __shared__ uint32_t epos[kScalexBlock];
  __shared__ uint8_t eval[kScalexBlock];
  __shared__ long long erange[2];
  const int64_t *row = table + (long long)kScalexCols * blockIdx.y;
  const long long raw = row[2];
  const long long b0 = (long long)blockIdx.x * kScalexBlock;
  if (b0 >= raw) return;
  const long long b1 = b0 + kScalexBlock < raw ? b0 + kScalexBlock : raw;
  const uint8_t *primary = staging + row[0] + kScalexHeader;
  const int codec = (int)row[3];
  const uint32_t palette = (uint32_t)row[4];
  const long long nexc = row[6];
  const uint8_t *pos = primary + row[5];  // u32 little-endian each, ascending
  const uint8_t *vals = pos + 4 * nexc;
  // this workgroup's exceptions: [lower_bound(b0), lower_bound(b1))
  if (threadIdx.x < 2) {
    const long long key = threadIdx.x == 0 ? b0 : b1;
    long long lo = 0, hi = nexc;
    while (lo < hi) {
      const long long mid = (lo + hi) >> 1;
      if ((long long)load_u32_le(pos + 4 * mid) < key) lo = mid + 1;
      else hi = mid;
    }
    erange[threadIdx.x] = lo;
  }
  __syncthreads();
  const long long e0 = erange[0];
  long long ne = erange[1] - e0;
  ne = ne < 0 ? 0 : (ne > kScalexBlock ? kScalexBlock : ne);  // bounded even if unsorted
  for (int q = threadIdx.x; q < ne; q += kScatterThreads) {
    epos[q] = load_u32_le(pos + 4 * (e0 + q));
    eval[q] = vals[e0 + q];
  }
  __syncthreads();
  const long long n0 = row[8], n1 = row[10];
  uint8_t *d0 = reinterpret_cast<uint8_t *>(row[7]);
  uint8_t *d1 = reinterpret_cast<uint8_t *>(row[9]);
  uint8_t *d2 = reinterpret_cast<uint8_t *>(row[11]);
  for (long long p = b0 + threadIdx.x; p < b1; p += kScatterThreads) {
    uint32_t v;
    if (codec == 0) v = primary[p];
    else if (codec == 1) v = palette >> (8 * ((primary[p >> 3] >> (p & 7)) & 1));
    else v = palette >> (8 * ((primary[p >> 2] >> (2 * (p & 3))) & 3));
    int lo = 0, hi = (int)ne;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((long long)epos[mid] < p) lo = mid + 1;
      else hi = mid;
    }
    if (lo < ne && (long long)epos[lo] == p) v = eval[lo];
    if (p < n0) d0[p] = (uint8_t)v;
    else if (p < n0 + n1) d1[p - n0] = (uint8_t)v;
    else d2[p - n0 - n1] = (uint8_t)v;
  }
}

}  // namespace glm

using namespace glm;

extern "C" int glm_scalex_decode(void *stream, const uint8_t *staging, int64_t staging_bytes,
                                 const int64_t *records, int n, int64_t *device_table) {
  glm::clear_error();
  GLM_REQUIRE(n >= 0 && staging_bytes >= 0, GLM_ERR_INVALID_ARGUMENT,
              "scalex_decode: negative record count or staging size");
  if (n == 0) return GLM_OK;
  GLM_REQUIRE(staging && records && device_table, GLM_ERR_INVALID_ARGUMENT,
              "scalex_decode: null pointer");
  long long max_raw = 0;
  for (int i = 0; i < n; ++i) {
    const int64_t *r = records + (long long)kScalexCols * i;
    const long long off = r[0], enc = r[1], raw = r[2], primary = r[5], exc = r[6];
    const int codec = (int)r[3];
    GLM_REQUIRE(off >= 0 && enc >= kScalexHeader && off + enc <= staging_bytes,
                GLM_ERR_INVALID_ARGUMENT, "scalex_decode: record %d is outside the staging buffer",
                i);
    GLM_REQUIRE(raw >= 1 && primary >= 0 && exc >= 0 && kScalexHeader + primary + 5 * exc == enc,
                GLM_ERR_INVALID_ARGUMENT, "scalex_decode: record %d has an inconsistent length",
                i);
    const long long want = codec == 0 ? raw : codec == 1 ? (raw + 7) / 8 : (raw + 3) / 4;
    GLM_REQUIRE(codec >= 0 && codec <= 2 && primary == want && (codec != 0 || exc == 0),
                GLM_ERR_INVALID_ARGUMENT, "scalex_decode: record %d has a bad codec or primary size",
                i);
    GLM_REQUIRE(r[8] >= 0 && r[10] >= 0 && r[12] >= 0 && r[8] + r[10] + r[12] == raw,
                GLM_ERR_INVALID_ARGUMENT, "scalex_decode: record %d destinations do not cover it",
                i);
    GLM_REQUIRE((r[8] == 0 || r[7]) && (r[10] == 0 || r[9]) && (r[12] == 0 || r[11]),
                GLM_ERR_INVALID_ARGUMENT, "scalex_decode: record %d has a null destination", i);
    max_raw = std::max(max_raw, raw);
  }
  const long long blocks = (max_raw + kScalexBlock - 1) / kScalexBlock;
  GLM_REQUIRE(blocks <= 0x7fffffffll, GLM_ERR_UNSUPPORTED_SHAPE, "scalex_decode: record too large");
  GLM_HIP_CHECK(hipMemcpyAsync(device_table, records, (size_t)n * kScalexCols * sizeof(int64_t),
                               hipMemcpyHostToDevice, (hipStream_t)stream));
  for (int first = 0; first < n; first += kMaxSegmentsPerLaunch) {
    const int count = std::min(kMaxSegmentsPerLaunch, n - first);
    hipLaunchKernelGGL(scalex_decode_kernel, dim3((unsigned)blocks, (unsigned)count),
                       dim3(kScatterThreads), 0, (hipStream_t)stream, staging,
                       device_table + (long long)kScalexCols * first);
    GLM_LAUNCH_CHECK("scalex_decode_kernel");
  }
  return GLM_OK;
}

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
    const int64_t *row = segments + (long long)glm::kScatterCols * i;
    GLM_REQUIRE(row[0] >= 0 && row[2] >= 0 && row[0] + row[2] <= staging_bytes,
                GLM_ERR_INVALID_ARGUMENT,
                "bank_scatter: segment %d [%lld, +%lld) is outside the %lld-byte staging buffer", i,
                (long long)row[0], (long long)row[2], (long long)staging_bytes);
    GLM_REQUIRE(row[2] == 0 || row[1] != 0, GLM_ERR_INVALID_ARGUMENT,
                "bank_scatter: segment %d has no destination", i);
    if (row[3] != 0) {
      const long long K = row[3], rows = K > 0 && K % 2 == 0 ? row[2] / (K / 2) : 0;
      GLM_REQUIRE(K > 0 && rows * (K / 2) == row[2] && glm::mxfp4_tiled(rows, K) &&
                      (row[1] & 15) == 0,
                  GLM_ERR_INVALID_ARGUMENT,
                  "bank_scatter: segment %d is not a tileable MXFP4 matrix (K %lld, %lld bytes: "
                  "rows %% 16 == 0 and K %% 128 == 0, a 16-byte aligned destination)",
                  i, K, (long long)row[2]);
    }
    max_bytes = std::max<long long>(max_bytes, row[2]);
  }
  if (max_bytes == 0) return GLM_OK;
  const long long blocks = (max_bytes + kScatterBlockBytes - 1) / kScatterBlockBytes;
  GLM_REQUIRE(blocks <= 0x7fffffffll, GLM_ERR_UNSUPPORTED_SHAPE, "bank_scatter: segment too large");
  GLM_HIP_CHECK(hipMemcpyAsync(device_table, segments,
                               (size_t)n * glm::kScatterCols * sizeof(int64_t),
                               hipMemcpyHostToDevice, (hipStream_t)stream));
  for (int first = 0; first < n; first += kMaxSegmentsPerLaunch) {
    const int count = std::min(kMaxSegmentsPerLaunch, n - first);
    hipLaunchKernelGGL(bank_scatter_kernel, dim3((unsigned)blocks, (unsigned)count),
                       dim3(kScatterThreads), 0, (hipStream_t)stream, staging,
                       device_table + (long long)glm::kScatterCols * first);
    GLM_LAUNCH_CHECK("bank_scatter_kernel");
  }
  return GLM_OK;
}

extern "C" int glm_mxfp4_is_tiled(int rows, int K) {
  return rows > 0 && K > 0 && glm::mxfp4_tiled(rows, K) ? 1 : 0;
}

extern "C" int glm_mxfp4_tile(void *stream, const uint8_t *src, uint8_t *dst, int64_t count,
                              int rows, int K) {
  glm::clear_error();
  GLM_REQUIRE(count >= 0 && rows >= 1 && K >= 32 && K % 32 == 0, GLM_ERR_INVALID_ARGUMENT,
              "mxfp4_tile: count %lld rows %d K %d (K a multiple of 32)", (long long)count, rows,
              K);
  if (count == 0) return GLM_OK;
  GLM_REQUIRE(src && dst, GLM_ERR_INVALID_ARGUMENT, "mxfp4_tile: null pointer");
  const long long bytes = count * (long long)rows * (K / 2);
  const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), d0 = reinterpret_cast<uintptr_t>(dst);
  GLM_REQUIRE(d0 + bytes <= s0 || s0 + bytes <= d0, GLM_ERR_INVALID_ARGUMENT,
              "mxfp4_tile: source and destination overlap");
  if (!glm::mxfp4_tiled(rows, K)) {  // this geometry stays row-major
    GLM_HIP_CHECK(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice,
                                 (hipStream_t)stream));
    return GLM_OK;
  }
  GLM_REQUIRE(((s0 | d0) & 15) == 0, GLM_ERR_INVALID_ARGUMENT,
              "mxfp4_tile: buffers must be 16-byte aligned");
  const long long pieces = bytes / 16;
  const long long blocks = std::min<long long>((pieces + glm::kScatterThreads - 1) /
                                               glm::kScatterThreads, 65536);
  hipLaunchKernelGGL(glm::mxfp4_tile_kernel, dim3((unsigned)blocks), dim3(glm::kScatterThreads), 0,
                     (hipStream_t)stream, src, dst, pieces, (long long)rows * (K / 32), K);
  GLM_LAUNCH_CHECK("mxfp4_tile_kernel");
  return GLM_OK;
}
