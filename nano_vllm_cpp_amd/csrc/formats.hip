// On-device Q8_0 format conversion: interleaved 34-byte GGUF blocks (fp16 scale,
// then 32 int8 values) into the two planes the GEMM and the split-plane gather
// read: w8 (32 bytes per block, contiguous) and ws (one fp16 scale per block).
//
// The reference splits on the host before upload (upload_q8_split,
// src/model.cpp:396-405, over the bytes load_q8_0 reads, src/gguf.cpp:353-362).
// Here the raw GGUF bytes go to HBM once and are split there; the conversion is
// a pure byte permutation, HBM-bound at 68 bytes per block.
//
// A workgroup takes kSplitBlocks consecutive blocks: 16-byte buffer loads stage
// the chunk in LDS (the 34-byte stride leaves the 32 value bytes of every other
// block 2 bytes off dword alignment), then each lane assembles 16-byte runs of
// w8 from dword-aligned LDS reads with a byte align, and packs two scales per
// dword of ws.
#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

// 256 blocks per workgroup (measured: 64..384 blocks all reach ~5.8 TB/s, 512 and
// more lose 7%); the loads carry the streaming (non-temporal) cache policy.
constexpr int kSplitBlocks = 256;
constexpr int kSplitBytes = kSplitBlocks * 34;    // 8704: a multiple of 16
constexpr int kSplitNt = 2;                       // buffer-load cache policy: non-temporal
constexpr int kSplitThreads = 256;

__global__ __launch_bounds__(kSplitThreads) void q8_0_split_kernel(const uint8_t* __restrict__ blocks,
                                                                   int64_t nblocks, uint8_t* __restrict__ w8,
                                                                   uint16_t* __restrict__ ws) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[kSplitBytes / 4];
  const int64_t b0 = (int64_t)blockIdx.x * kSplitBlocks;
  const int nb = (int)min<int64_t>(kSplitBlocks, nblocks - b0);
  const int bytes = nb * 34;
  // Loads wholly past the last block read as zero (never stored).  A load that
  // straddles the end would read zero as a whole, so the one 16-byte chunk that
  // does (34 nb is even but not always a multiple of 16) is read 2 bytes at a time.
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(blocks + b0 * 34), (short)0, bytes, 0x00020000);
  for (int i = threadIdx.x; i < kSplitBytes / 16; i += kSplitThreads) {
    u32x4 v;
    if (16 * i + 16 <= bytes || 16 * i >= bytes) {
      v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(16 * i), 0, kSplitNt));
    } else {
      uint32_t d[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        d[q] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (uint32_t)(16 * i + 4 * q), 0, 0) |
               ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (uint32_t)(16 * i + 4 * q + 2), 0, 0) << 16);
      v = u32x4{d[0], d[1], d[2], d[3]};
    }
    *reinterpret_cast<u32x4*>(&lds[4 * i]) = v;
  }
  __syncthreads();

  // w8: output run o = 16 bytes = half h of block b; its source starts at byte
  // 34 b + 2 + 16 h, which is dword-aligned for odd b and 2 bytes past for even b.
  for (int o = threadIdx.x; o < 2 * nb; o += kSplitThreads) {
    const int b = o >> 1, h = o & 1;
    const int s = 34 * b + 2 + 16 * h;
    const uint32_t* p = &lds[s >> 2];
    u32x4 v;
    if (s & 2) {
      const uint32_t w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
      v = u32x4{__builtin_amdgcn_alignbyte(w1, w0, 2), __builtin_amdgcn_alignbyte(w2, w1, 2),
                __builtin_amdgcn_alignbyte(w3, w2, 2), __builtin_amdgcn_alignbyte(w4, w3, 2)};
    } else {
      v = u32x4{p[0], p[1], p[2], p[3]};
    }
    st16_nt(w8 + (b0 + b) * 32 + 16 * h, v);
  }

  // ws: the scales of blocks 2j and 2j+1 (LDS bytes 68 j and 68 j + 34) packed
  // into one dword; a lone last scale is stored by itself.
  const uint16_t* l16 = reinterpret_cast<const uint16_t*>(lds);
  for (int j = threadIdx.x; 2 * j < nb; j += kSplitThreads) {
    const uint32_t lo = l16[34 * j], hi = l16[34 * j + 17];
    if (2 * j + 1 < nb)
      *reinterpret_cast<uint32_t*>(ws + b0 + 2 * j) = lo | (hi << 16);
    else
      ws[b0 + 2 * j] = (uint16_t)lo;
  }
}

}  // namespace nvf

extern "C" int nvf_q8_0_split_blocks(const uint8_t* blocks, int64_t nblocks, int8_t* w8, uint16_t* ws,
                                     void* stream) {
  using namespace nvf;
  if (nblocks < 0) return fail(NVF_ERR_INVALID, "nvf_q8_0_split_blocks: nblocks %lld < 0", (long long)nblocks);
  if (nblocks == 0) return NVF_OK;
  if (!blocks || !w8 || !ws) return fail(NVF_ERR_INVALID, "nvf_q8_0_split_blocks: NULL pointer");
  if (!aligned16(blocks) || !aligned16(w8) || (reinterpret_cast<uintptr_t>(ws) & 3u))
    return fail(NVF_ERR_INVALID,
                "nvf_q8_0_split_blocks: blocks and w8 must be 16-byte aligned, ws 4-byte aligned");
  const int64_t wgs = (nblocks + kSplitBlocks - 1) / kSplitBlocks;
  if (wgs > INT32_MAX) return fail(NVF_ERR_INVALID, "nvf_q8_0_split_blocks: too many blocks");
  q8_0_split_kernel<<<dim3((unsigned)wgs), kSplitThreads, 0, as_stream(stream)>>>(
      blocks, nblocks, reinterpret_cast<uint8_t*>(w8), ws);
  return launch_status("q8_0_split_blocks");
}
