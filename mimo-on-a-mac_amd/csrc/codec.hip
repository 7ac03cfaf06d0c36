// MXFP4 codec, seeded random pools, activation hi/lo split, bf16 sigmoid table, error state.
#include <mutex>
#include <string>
#include <string.h>
#include <vector>

#include "device.h"
#include "host.h"
#include "router.h"
#include "sigmoid_table.h"

namespace mimo {

// ------------------------------------------------------------------ error state
static thread_local std::string g_err;
int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}
void clear_error() { g_err.clear(); }

// ------------------------------------------------------------------ opt-in kernel timing
struct ProfRec {
  const char* name;
  hipEvent_t a, b;
  bool owns_a;          // false when a is the previous record's end event (chained)
};
static std::mutex g_prof_mu;
static bool g_prof_on = false;
static std::vector<ProfRec> g_prof;
static std::vector<hipEvent_t> g_prof_pool;
static const char* g_prof_open = nullptr;
static hipEvent_t g_prof_open_ev;
static bool g_prof_open_owns = true;
// Within one multi-kernel entry point (ProfChain), a kernel's begin is the previous kernel's end event on the
// same stream: one event per launch, so the timing adds no begin packet of its own.
static int g_prof_chain = 0;
static hipEvent_t g_prof_last_end = nullptr;
static hipStream_t g_prof_last_stream = nullptr;
static thread_local int t_prof_suspend = 0;

void prof_suspend(bool on) { t_prof_suspend += on ? 1 : -1; }

static hipEvent_t prof_event() {
  if (!g_prof_pool.empty()) {
    hipEvent_t e = g_prof_pool.back();
    g_prof_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void prof_begin(hipStream_t st, const char* name) {
  if (!g_prof_on || t_prof_suspend) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (g_prof_chain && g_prof_last_end && g_prof_last_stream == st) {
    g_prof_open = name;
    g_prof_open_ev = g_prof_last_end;
    g_prof_open_owns = false;
    return;
  }
  hipEvent_t e = prof_event();
  if (!e) return;
  if (hipEventRecord(e, st) != hipSuccess) {   // timing is best effort: this launch goes unrecorded
    g_prof_pool.push_back(e);
    return;
  }
  g_prof_open = name;
  g_prof_open_ev = e;
  g_prof_open_owns = true;
}

void prof_end(hipStream_t st) {
  if (!g_prof_on || t_prof_suspend) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (!g_prof_open) return;
  hipEvent_t e = prof_event();
  if (!e || hipEventRecord(e, st) != hipSuccess) {   // drop this launch's record; the chain restarts
    if (e) g_prof_pool.push_back(e);
    if (g_prof_open_owns) g_prof_pool.push_back(g_prof_open_ev);
    g_prof_open = nullptr;
    g_prof_last_end = nullptr;
    return;
  }
  g_prof.push_back({g_prof_open, g_prof_open_ev, e, g_prof_open_owns});
  g_prof_open = nullptr;
  g_prof_last_end = e;
  g_prof_last_stream = st;
}

void prof_chain(bool on) {
  if (!g_prof_on || t_prof_suspend) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_chain += on ? 1 : -1;
  if (on && g_prof_chain == 1) g_prof_last_end = nullptr;     // the chain starts with a fresh begin event
}

// ------------------------------------------------------------------ seeded normal generator
// Element i of stream `seed`: splitmix64 of (seed, i) gives two 24-bit uniforms, Box-Muller gives N(0,1).
__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i) {
#pragma clang fp contract(off)
  uint64_t z = seed * 0xD1B54A32D192ED03ull + i * 0x9E3779B97F4A7C15ull + 0x632BE59BD9B4E019ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  float u1 = ((float)(uint32_t)(z >> 40) + 0.5f) * (1.0f / 16777216.0f);
  float u2 = (float)(uint32_t)(z & 0xFFFFFFu) * (1.0f / 16777216.0f);
  float r = sqrtf(-2.0f * logf(u1));
  return r * cosf(6.283185307179586f * u2);
}

// ------------------------------------------------------------------ MXFP4 block quantiser
// 32 values (fp32, bf16-valued) -> 4 packed words + E8M0 byte.  OCP: X = floor(log2 amax) - 2.
__device__ __forceinline__ void quant_block_mxfp4(const float* v, uint32_t* words, uint8_t* sbyte) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
  int X;
  if (amax == 0.0f) {
    X = -127;
  } else {
    uint32_t E = (__float_as_uint(amax) >> 23) & 0xFF;
    X = E == 0 ? -127 : (int)E - 127 - 2;
    X = X < -127 ? -127 : (X > 127 ? 127 : X);
  }
  float inv = exp2i(-X);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float x = v[w * 8 + j];
      uint32_t mag = e2m1_mag_code(fabsf(x) * inv);
      uint32_t code = mag | ((mag != 0u && x < 0.0f) ? 8u : 0u);
      word |= code << (4 * j);
    }
    words[w] = word;
  }
  *sbyte = (uint8_t)(X + 127);
}

__global__ void quantize_mxfp4_kernel(const uint16_t* __restrict__ w, int64_t nblocks, uint32_t* __restrict__ q,
                                      uint8_t* __restrict__ s) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint4* src = reinterpret_cast<const uint4*>(w + b * 32);
  float v[32];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint4 d = src[c];
    uint32_t parts[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[c * 8 + 2 * j] = __uint_as_float(parts[j] << 16);
      v[c * 8 + 2 * j + 1] = __uint_as_float(parts[j] & 0xFFFF0000u);
    }
  }
  uint32_t words[4];
  uint8_t sb;
  quant_block_mxfp4(v, words, &sb);
  reinterpret_cast<uint4*>(q)[b] = make_uint4(words[0], words[1], words[2], words[3]);
  s[b] = sb;
}

__global__ void fill_random_mxfp4_kernel(uint64_t seed, float stddev, int64_t nblocks, uint32_t* __restrict__ q,
                                         uint8_t* __restrict__ s) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  float v[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) v[j] = round_bf16(normal_at(seed, (uint64_t)(b * 32 + j)) * stddev);
  uint32_t words[4];
  uint8_t sb;
  quant_block_mxfp4(v, words, &sb);
  reinterpret_cast<uint4*>(q)[b] = make_uint4(words[0], words[1], words[2], words[3]);
  s[b] = sb;
}

__global__ void random_bf16_kernel(uint64_t seed, float stddev, int64_t n, uint16_t* __restrict__ out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = f32_to_bf16(normal_at(seed, (uint64_t)i) * stddev);
}

__global__ void dequantize_mxfp4_kernel(const uint32_t* __restrict__ q, const uint8_t* __restrict__ s,
                                        int64_t nwords, float* __restrict__ out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nwords) return;
  uint32_t word = q[i];
  uint32_t sb = s[i >> 2];
  float scale = sb == 255u ? __uint_as_float(0x7FC00000u) : exp2i((int)sb - 127);
  const float tab[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  float4 lo, hi;
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t c = (word >> (4 * j)) & 0xFu;
    float m = tab[c & 7u] * scale;
    r[j] = (c & 8u) ? -m : m;
  }
  lo = make_float4(r[0], r[1], r[2], r[3]);
  hi = make_float4(r[4], r[5], r[6], r[7]);
  reinterpret_cast<float4*>(out)[2 * i] = lo;
  reinterpret_cast<float4*>(out)[2 * i + 1] = hi;
}

// ------------------------------------------------------------------ activation hi/lo split
__global__ void quantize_fp8_hilo_kernel(const uint16_t* __restrict__ x, int64_t nblocks, uint8_t* __restrict__ hi,
                                         uint8_t* __restrict__ hs, uint8_t* __restrict__ lo,
                                         uint8_t* __restrict__ ls, int32_t* zero_status) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (zero_status && b == 0) *zero_status = 0;
  if (b >= nblocks) return;
  const uint4* src = reinterpret_cast<const uint4*>(x + b * 32);
  float v[32];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint4 d = src[c];
    uint32_t parts[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[c * 8 + 2 * j] = __uint_as_float(parts[j] << 16);
      v[c * 8 + 2 * j + 1] = __uint_as_float(parts[j] & 0xFFFF0000u);
    }
  }
  uint32_t hw[8], lw[8];
  uint8_t hsb, lsb;
  quant_block_fp8_hilo(v, hw, lw, &hsb, &lsb);
  uint4* H = reinterpret_cast<uint4*>(hi + b * 32);
  uint4* L = reinterpret_cast<uint4*>(lo + b * 32);
  H[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  H[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
  L[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  L[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
  hs[b] = hsb;
  ls[b] = lsb;
}

int launch_quantize_fp8_hilo(const uint16_t* x, int64_t rows, int64_t cols, uint8_t* hi, uint8_t* hs, uint8_t* lo,
                             uint8_t* ls, hipStream_t st, int32_t* zero_status) {
  int64_t nb = rows * (cols / 32);
  if (nb == 0) return MIMO_OK;
  ProfScope p(st, "quantize_fp8_hilo");
  quantize_fp8_hilo_kernel<<<(int)((nb + 255) / 256), 256, 0, st>>>(x, nb, hi, hs, lo, ls, zero_status);
  return check_launch("quantize_fp8_hilo");
}

// ------------------------------------------------------------------ bf16 sigmoid table
// The table is data in the code object (evaluated by the compiler, sigmoid_table.h): nothing is built or
// synchronised at run time, so any call, including the first prefill of a process under graph capture, only
// looks up its device address (no stream work).
static __device__ sigtab_gen::Table g_sigtab = sigtab_gen::make();

static std::mutex g_sig_mu;
static const uint16_t* g_sig_ptr[64];

const uint16_t* sigtab_device(int* err) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    *err = set_error(MIMO_ERR_HIP, "hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_sig_mu);
  if (!g_sig_ptr[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_sigtab));
    if (e != hipSuccess) {
      *err = set_error(MIMO_ERR_HIP, "hipGetSymbolAddress(sigtab): %s", hipGetErrorString(e));
      return nullptr;
    }
    g_sig_ptr[dev] = static_cast<const uint16_t*>(p);
  }
  *err = MIMO_OK;
  return g_sig_ptr[dev];
}

}  // namespace mimo

using namespace mimo;

extern "C" {

int mimo_abi_version(void) { return MIMO_ABI_VERSION; }

int mimo_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  for (auto& r : g_prof) {
    if (r.owns_a) g_prof_pool.push_back(r.a);
    g_prof_pool.push_back(r.b);
  }
  g_prof.clear();
  g_prof_open = nullptr;
  g_prof_last_end = nullptr;
  g_prof_chain = 0;
  g_prof_on = on != 0;
  return MIMO_OK;
}

int mimo_profile_read(int max_kernels, char* names, float* total_ms, int* launches) {
  MIMO_REQUIRE(max_kernels >= 0 && (max_kernels == 0 || (names && total_ms && launches)), MIMO_ERR_ARG,
               "profile_read: null pointer");
  std::lock_guard<std::mutex> lk(g_prof_mu);
  std::vector<const char*> keys;
  std::vector<double> tot;
  std::vector<int> cnt;
  for (auto& r : g_prof) {
    if (hipEventSynchronize(r.b) != hipSuccess) return set_error(MIMO_ERR_HIP, "profile_read: event sync failed");
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return set_error(MIMO_ERR_HIP, "profile_read: elapsed");
    size_t j = 0;
    while (j < keys.size() && strcmp(keys[j], r.name) != 0) ++j;
    if (j == keys.size()) { keys.push_back(r.name); tot.push_back(0.0); cnt.push_back(0); }
    tot[j] += ms;
    cnt[j] += 1;
  }
  int n = (int)keys.size() < max_kernels ? (int)keys.size() : max_kernels;
  for (int j = 0; j < n; ++j) {
    strncpy(names + 64 * j, keys[j], 63);
    names[64 * j + 63] = 0;
    total_ms[j] = (float)tot[j];
    launches[j] = cnt[j];
  }
  return (int)keys.size();
}
const char* mimo_last_error(void) { return g_err.c_str(); }

static int grid_for(int64_t n, int threads) { return (int)((n + threads - 1) / threads); }

int mimo_quantize_mxfp4(const uint16_t* w, int64_t rows, int64_t cols, uint32_t* q, uint8_t* s, void* stream) {
  MIMO_REQUIRE(w && q && s, MIMO_ERR_ARG, "quantize_mxfp4: null pointer");
  MIMO_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, MIMO_ERR_SHAPE, "quantize_mxfp4: cols %% 32 != 0");
  MIMO_REQUIRE(aligned16(w) && aligned16(q), MIMO_ERR_ALIGN, "quantize_mxfp4: 16-byte alignment");
  int64_t nb = rows * (cols / 32);
  if (nb == 0) return MIMO_OK;
  quantize_mxfp4_kernel<<<grid_for(nb, 256), 256, 0, as_stream(stream)>>>(w, nb, q, s);
  return check_launch("quantize_mxfp4");
}

int mimo_dequantize_mxfp4(const uint32_t* q, const uint8_t* s, int64_t rows, int64_t cols, float* out,
                          void* stream) {
  MIMO_REQUIRE(q && s && out, MIMO_ERR_ARG, "dequantize_mxfp4: null pointer");
  MIMO_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, MIMO_ERR_SHAPE, "dequantize_mxfp4: cols %% 32 != 0");
  MIMO_REQUIRE(aligned16(out), MIMO_ERR_ALIGN, "dequantize_mxfp4: 16-byte alignment");
  int64_t nw = rows * (cols / 8);
  if (nw == 0) return MIMO_OK;
  dequantize_mxfp4_kernel<<<grid_for(nw, 256), 256, 0, as_stream(stream)>>>(q, s, nw, out);
  return check_launch("dequantize_mxfp4");
}

int mimo_random_bf16(uint64_t seed, float stddev, int64_t n, uint16_t* out, void* stream) {
  MIMO_REQUIRE(out, MIMO_ERR_ARG, "random_bf16: null pointer");
  MIMO_REQUIRE(n >= 0, MIMO_ERR_SHAPE, "random_bf16: n < 0");
  if (n == 0) return MIMO_OK;
  random_bf16_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(seed, stddev, n, out);
  return check_launch("random_bf16");
}

int mimo_fill_random_mxfp4(uint64_t seed, float stddev, int64_t rows, int64_t cols, uint32_t* q, uint8_t* s,
                           void* stream) {
  MIMO_REQUIRE(q && s, MIMO_ERR_ARG, "fill_random_mxfp4: null pointer");
  MIMO_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, MIMO_ERR_SHAPE, "fill_random_mxfp4: cols %% 32 != 0");
  MIMO_REQUIRE(aligned16(q), MIMO_ERR_ALIGN, "fill_random_mxfp4: 16-byte alignment");
  int64_t nb = rows * (cols / 32);
  if (nb == 0) return MIMO_OK;
  fill_random_mxfp4_kernel<<<grid_for(nb, 256), 256, 0, as_stream(stream)>>>(seed, stddev, nb, q, s);
  return check_launch("fill_random_mxfp4");
}

int mimo_quantize_fp8_hilo(const uint16_t* x, int64_t rows, int64_t cols, uint8_t* hi, uint8_t* hs, uint8_t* lo,
                           uint8_t* ls, void* stream) {
  MIMO_REQUIRE(x && hi && hs && lo && ls, MIMO_ERR_ARG, "quantize_fp8_hilo: null pointer");
  MIMO_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, MIMO_ERR_SHAPE, "quantize_fp8_hilo: cols %% 32 != 0");
  MIMO_REQUIRE(aligned16(x) && aligned16(hi) && aligned16(lo), MIMO_ERR_ALIGN, "quantize_fp8_hilo: alignment");
  return launch_quantize_fp8_hilo(x, rows, cols, hi, hs, lo, ls, as_stream(stream));
}

int mimo_sigmoid_table(uint16_t* out, void* stream) {
  MIMO_REQUIRE(out, MIMO_ERR_ARG, "sigmoid_table: null pointer");
  int err;
  const uint16_t* tab = sigtab_device(&err);
  if (!tab) return err;
  MIMO_HIP(hipMemcpyAsync(out, tab, 65536 * sizeof(uint16_t), hipMemcpyDeviceToDevice, as_stream(stream)));
  return MIMO_OK;
}

}  // extern "C"
