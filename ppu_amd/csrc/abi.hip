// ABI version query (the value must match Q35_ABI_VERSION in include/q35.h)
// and the cache reset: every state tensor of a reused KV / linear-attention
// cache zeroed by one launch instead of one fill kernel per tensor.
#include "q35_common.hpp"

namespace {

constexpr int kZeroMax = 32;  // buffers per launch (kernel argument struct)

struct ZeroArgs {
  uint8_t* p[kZeroMax];
  long long nbytes[kZeroMax];
};

// Grid (chunks, buffers): buffer blockIdx.y is cleared with 16-byte stores
// (grid-stride), its last nbytes % 16 bytes byte by byte. Buffers start
// 16-byte aligned (checked on the host).
__global__ __launch_bounds__(256) void zero_buffers(const ZeroArgs a) {
  uint8_t* p = a.p[blockIdx.y];
  const long long n = a.nbytes[blockIdx.y];
  const long long n16 = n & ~15ll;
  const q35_u32x4 z = {0u, 0u, 0u, 0u};
  for (long long off = ((long long)blockIdx.x * 256 + threadIdx.x) * 16; off < n16;
       off += (long long)gridDim.x * 256 * 16)
    *reinterpret_cast<q35_u32x4*>(p + off) = z;
  if (blockIdx.x == 0 && threadIdx.x < n - n16) p[n16 + threadIdx.x] = 0;
}

}  // namespace

extern "C" {

int q35_abi_version(void) { return 1; }

// Zero n device buffers (host arrays of pointers and byte counts; each
// pointer 16-byte aligned). Replaces the per-tensor zero_() calls of
// Transformers' Cache.reset() for the caches the generation loop reuses
// (evaluation_wrapper.py:350-352).
int q35_zero_buffers(void* const* ptrs, const long long* nbytes, int n, hipStream_t stream) {
  Q35_CHECK_ARG(n >= 0 && (n == 0 || (ptrs && nbytes)));
  for (int b0 = 0; b0 < n; b0 += kZeroMax) {
    const int cnt = min(kZeroMax, n - b0);
    ZeroArgs a{};
    long long most = 0;
    for (int i = 0; i < cnt; ++i) {
      Q35_CHECK_ARG(nbytes[b0 + i] >= 0 && (nbytes[b0 + i] == 0 || q35_aligned16(ptrs[b0 + i])));
      a.p[i] = (uint8_t*)ptrs[b0 + i];
      a.nbytes[i] = nbytes[b0 + i];
      most = nbytes[b0 + i] > most ? nbytes[b0 + i] : most;
    }
    if (most == 0) continue;
    const long long chunks = (most + 256 * 16 - 1) / (256 * 16);
    const unsigned gx = (unsigned)(chunks < 1024 ? chunks : 1024);
    zero_buffers<<<dim3(gx, (unsigned)cnt), 256, 0, stream>>>(a);
    const int e = q35_last_error();
    if (e) return e;
  }
  return 0;
}

}  // extern "C"
