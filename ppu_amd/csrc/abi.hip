// ABI version query (the value must match Q35_ABI_VERSION in include/q35.h),
// the cache reset (every state tensor of a reused KV / linear-attention cache
// zeroed by one launch instead of one fill kernel per tensor) and the HBM
// read-rate probe that the decode GEMVs are measured against.
#include "q35_common.hpp"

namespace {

constexpr int kZeroMax = 128;  // buffers per launch (kernel argument struct, 2 KiB)

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

// Read-rate probe: every 16-byte group of p read once with non-temporal
// loads (the GEMV weight-stream load), grid-stride over a persistent grid,
// 8 loads per lane in flight, an XOR fold so no load is dead; one word per
// thread. 8 loads per lane on one workgroup of 4 waves per CU was the
// fastest of 36 shapes (grid size x loads in flight x row-chunked order)
// over the 1 GB lm_head weight.
constexpr int kReadU = 8;
__global__ __launch_bounds__(256) void stream_read(const uint8_t* __restrict__ p, long long n16,
                                                   uint32_t* __restrict__ out) {
  const long long stride = (long long)gridDim.x * 256;
  uint32_t acc = 0;
  // The last sweep issues its loads together too: an index past the end
  // reads the lane's own first group of the sweep again (clamped, no branch
  // to split the batch, no line every lane hits) and is not folded in.
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += kReadU * stride) {
    uint4 v[kReadU];
#pragma unroll
    for (int u = 0; u < kReadU; ++u) {
      const long long j = i + u * stride;
      v[u] = ld_stream16(p + (j < n16 ? j : i) * 16);
    }
#pragma unroll
    for (int u = 0; u < kReadU; ++u)
      acc ^= i + u * stride < n16 ? v[u].x ^ v[u].y ^ v[u].z ^ v[u].w : 0u;
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc;
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

}  // namespace

extern "C" {

int q35_abi_version(void) { return 5; }

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

// Read nbytes (a multiple of 16, p 16-byte aligned) once; out receives one
// XOR word per thread (out_words >= 256 * workgroups; workgroups = the CU
// count, written to *workgroups_out when it is not null).
int q35_stream_read(const void* p, long long nbytes, void* out, long long out_words, int* workgroups_out,
                    hipStream_t stream) {
  Q35_CHECK_ARG(p && out && nbytes > 0 && nbytes % 16 == 0 && q35_aligned16(p));
  const int blocks = device_cus();
  Q35_CHECK_ARG(out_words >= (long long)blocks * 256);
  if (workgroups_out) *workgroups_out = blocks;
  stream_read<<<blocks, 256, 0, stream>>>((const uint8_t*)p, nbytes / 16, (uint32_t*)out);
  return q35_last_error();
}

// The same probe as one round of requests: enough workgroups that no lane
// issues more than kReadU loads (at least one workgroup per CU while the
// buffer gives every lane a load), so every byte is requested at once. The
// read floor of a small kernel: one launch that must fetch nbytes.
int q35_stream_read_round(const void* p, long long nbytes, void* out, long long out_words,
                          int* workgroups_out, hipStream_t stream) {
  Q35_CHECK_ARG(p && out && nbytes > 0 && nbytes % 16 == 0 && q35_aligned16(p));
  const long long n16 = nbytes / 16;
  const long long one_round = (n16 + 256ll * kReadU - 1) / (256ll * kReadU);
  const long long per_cu = (n16 + 255) / 256;
  const long long spread = per_cu < device_cus() ? per_cu : device_cus();
  const long long blocks = one_round > spread ? one_round : spread;
  Q35_CHECK_ARG(blocks < (1ll << 31) / 256 && out_words >= blocks * 256);
  if (workgroups_out) *workgroups_out = (int)blocks;
  stream_read<<<(unsigned)blocks, 256, 0, stream>>>((const uint8_t*)p, n16, (uint32_t*)out);
  return q35_last_error();
}

}  // extern "C"
