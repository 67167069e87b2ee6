// Flat stream copy: the bandwidth ceiling of a streaming kernel's access
// style on this device, as a yardstick next to each oracle kernel.
//
// Reads `read_bytes` from src and writes `write_bytes` to dst in one launch,
// in the access style of the oracle kernels: 16-byte non-temporal loads and
// stores, each wave64 moving one contiguous 1 KiB chunk of each buffer,
// 4 waves per 256-thread workgroup, a one-shot grid over
// max(read, write) / 1 KiB chunks in memory order.  Chunk i of dst receives
// chunk i of src where both exist (a plain copy when the sizes are equal);
// where only src exists the loaded value feeds a store that never fires for
// finite data, so the load is kept without adding writes; where only dst
// exists a constant is written.
//
// HBM-bound: algorithmic bytes = read_bytes + write_bytes.
//
// hipo_flat_copy2: the same for two input and two output streams moved
// chunk by chunk in lockstep (the residual LayerNorm's x, residual -> h, y),
// a pattern a one-stream copy does not share.
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kCopyWaves = 4;
constexpr int kChunk = kWave * 16;  // bytes per wave per buffer

__global__ __launch_bounds__(kCopyWaves * kWave) void flat_copy_chunks(
    const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
    uint64_t read_chunks, uint64_t write_chunks) {
  const uint64_t chunk = static_cast<uint64_t>(blockIdx.x) * kCopyWaves + (threadIdx.x >> 6);
  const uint64_t idx = chunk * kWave + (threadIdx.x & (kWave - 1));
  u32x4_t v = {0x3f800000u, 0x3f800000u, 0x3f800000u, 0x3f800000u};
  const bool rd = chunk < read_chunks;
  if (rd) v = __builtin_nontemporal_load(src + idx);
  if (chunk < write_chunks) {
    __builtin_nontemporal_store(v, dst + idx);
  } else if (rd && (v[0] & v[1] & v[2] & v[3]) == 0xffffffffu) {
    // All-ones words are NaNs: finite data never takes this store.
    __builtin_nontemporal_store(v, dst + (threadIdx.x & (kWave - 1)));
  }
}

// Two streams in, two out: wave chunk i moves 1 KiB of src0 to dst0 and 1
// KiB of src1 to dst1, all four accesses of a lane issued together.
__global__ __launch_bounds__(kCopyWaves * kWave) void flat_copy2_chunks(
    const u32x4_t* __restrict__ src0, const u32x4_t* __restrict__ src1,
    u32x4_t* __restrict__ dst0, u32x4_t* __restrict__ dst1, uint64_t chunks) {
  const uint64_t chunk = static_cast<uint64_t>(blockIdx.x) * kCopyWaves + (threadIdx.x >> 6);
  if (chunk >= chunks) return;
  const uint64_t idx = chunk * kWave + (threadIdx.x & (kWave - 1));
  const u32x4_t a = __builtin_nontemporal_load(src0 + idx);
  const u32x4_t b = __builtin_nontemporal_load(src1 + idx);
  __builtin_nontemporal_store(a, dst0 + idx);
  __builtin_nontemporal_store(b, dst1 + idx);
}

}  // namespace
}  // namespace hipo

extern "C" int hipo_flat_copy(const void* src, int64_t read_bytes, void* dst,
                              int64_t write_bytes, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(read_bytes >= 0 && write_bytes >= kChunk,
               "flat_copy: write_bytes must be at least %d", kChunk);
  HIPO_REQUIRE(read_bytes % kChunk == 0 && write_bytes % kChunk == 0,
               "flat_copy: sizes must be multiples of %d bytes", kChunk);
  HIPO_REQUIRE(dst && (src || read_bytes == 0), "flat_copy: null pointer");
  HIPO_REQUIRE(aligned16(src) && aligned16(dst), "flat_copy: pointers must be 16-byte aligned");
  const uint64_t rc = static_cast<uint64_t>(read_bytes) / kChunk;
  const uint64_t wc = static_cast<uint64_t>(write_bytes) / kChunk;
  const uint64_t chunks = rc > wc ? rc : wc;
  const uint64_t blocks = (chunks + kCopyWaves - 1) / kCopyWaves;
  HIPO_REQUIRE(blocks < (uint64_t{1} << 31), "flat_copy: too large");
  flat_copy_chunks<<<dim3(static_cast<unsigned>(blocks)), dim3(kCopyWaves * kWave), 0,
                     stream>>>(static_cast<const u32x4_t*>(src), static_cast<u32x4_t*>(dst),
                               rc, wc);
  return check_launch("flat_copy");
}

extern "C" int hipo_flat_copy2(const void* src0, const void* src1, void* dst0, void* dst1,
                               int64_t bytes, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(bytes >= kChunk && bytes % kChunk == 0,
               "flat_copy2: bytes must be a positive multiple of %d", kChunk);
  HIPO_REQUIRE(src0 && src1 && dst0 && dst1, "flat_copy2: null pointer");
  HIPO_REQUIRE(aligned16(src0) && aligned16(src1) && aligned16(dst0) && aligned16(dst1),
               "flat_copy2: pointers must be 16-byte aligned");
  const uint64_t chunks = static_cast<uint64_t>(bytes) / kChunk;
  const uint64_t blocks = (chunks + kCopyWaves - 1) / kCopyWaves;
  HIPO_REQUIRE(blocks < (uint64_t{1} << 31), "flat_copy2: too large");
  flat_copy2_chunks<<<dim3(static_cast<unsigned>(blocks)), dim3(kCopyWaves * kWave), 0,
                      stream>>>(static_cast<const u32x4_t*>(src0),
                                static_cast<const u32x4_t*>(src1), static_cast<u32x4_t*>(dst0),
                                static_cast<u32x4_t*>(dst1), chunks);
  return check_launch("flat_copy2");
}
