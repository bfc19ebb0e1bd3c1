// C-ABI runtime of libnspeech_rocm.so: code-object loading, argument
// validation, kernel selection and launch for every entry point declared in
// include/nspeech_rocm.h.
//
// The kernels live in one gfx950 code object per kernel unit
// (kernels/<unit>.hip), embedded in this library (nsr_embed.S) and loaded
// per device with hipModuleLoadData on first use. Every kernel has a
// compile-time id (KId, from nsr_kernels.def); all of a device's kernel
// handles are resolved when its modules are loaded, so a launch is an index
// into a per-device table and hipModuleLaunchKernel on the caller's stream:
// no name building, lock or lookup per call. This replaces the reference's
// Metal pipeline loading and dispatch (src/triton_kernels.rs:1401,
// kernels/out/generated/triton_metal_gen.rs:39-106) and its per-call encoder
// setup (src/triton_kernels.rs:312-1423).
#include "nspeech_rocm.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../nsr_kargs.h"
#include "nsr_scratch.h"

// Embedded code objects, one per kernel unit (nsr_embed.S).
extern "C" const unsigned char nsr_co_q8_0_gather[];
extern "C" const unsigned char nsr_co_layernorm[];
extern "C" const unsigned char nsr_co_rotary[];
extern "C" const unsigned char nsr_co_adain_snake[];
extern "C" const unsigned char nsr_co_elementwise[];
extern "C" const unsigned char nsr_co_gemv_q8[];
extern "C" const unsigned char nsr_co_conv1d[];
extern "C" const unsigned char nsr_co_attention[];
extern "C" const unsigned char nsr_co_istft[];
extern "C" const unsigned char nsr_co_calib[];

namespace {

enum UnitId { U_q8_0_gather, U_layernorm, U_rotary, U_adain_snake, U_elementwise, U_gemv_q8, U_conv1d,
              U_attention, U_istft, U_calib, kNumUnits };

struct Unit {
  const char* name;
  const unsigned char* image;
};
const Unit kUnits[kNumUnits] = {{"q8_0_gather", nsr_co_q8_0_gather},
                                {"layernorm", nsr_co_layernorm},
                                {"rotary", nsr_co_rotary},
                                {"adain_snake", nsr_co_adain_snake},
                                {"elementwise", nsr_co_elementwise},
                                {"gemv_q8", nsr_co_gemv_q8},
                                {"conv1d", nsr_co_conv1d},
                                {"attention", nsr_co_attention},
                                {"istft", nsr_co_istft},
                                {"calib", nsr_co_calib}};

// Kernel ids: K_<kernel name>, in nsr_kernels.def order; K_NONE marks a
// variant that is not built.
enum KId : int {
  K_NONE = -1,
#define NSR_KERNEL(unit, name) K_##name,
#include "nsr_kernels.def"
#undef NSR_KERNEL
  K_COUNT
};

struct KernelInfo {
  UnitId unit;
  const char* name;
};
const KernelInfo kKernels[K_COUNT] = {
#define NSR_KERNEL(unit, name) {U_##unit, #name},
#include "nsr_kernels.def"
#undef NSR_KERNEL
};

constexpr int kMaxDevices = 64;
thread_local std::string g_last_error;

nsr_status fail(nsr_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

struct DeviceModule {
  std::once_flag once;
  nsr_status status = NSR_ERR_NOT_INIT;
  std::string error;
  hipModule_t modules[kNumUnits] = {};
  hipFunction_t fn[K_COUNT] = {};
  std::atomic<int> occupancy[K_COUNT] = {};  // workgroups per CU, for kernels launched with one shape (0: unknown)
  int max_lds = 0;
  int n_cu = 0;
};

DeviceModule g_dev[kMaxDevices];
std::mutex g_path_mu;
std::string g_code_object_path;  // empty: embedded image

void load_module(DeviceModule& dm, int dev) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) {
    dm.error = std::string("hipGetDeviceProperties: ") + hipGetErrorString(e);
    dm.status = NSR_ERR_HIP;
    return;
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    dm.error = std::string("device ") + std::to_string(dev) + " is " + prop.gcnArchName +
               "; this library carries gfx950 code only";
    dm.status = NSR_ERR_NOT_INIT;
    return;
  }
  std::string path;
  {
    std::lock_guard<std::mutex> lk(g_path_mu);
    path = g_code_object_path;
  }
  for (int u = 0; u < kNumUnits; ++u) {
    const std::string file = path + "/nsr_" + kUnits[u].name + "_gfx950.hsaco";
    if (path.empty()) {
      e = hipModuleLoadData(&dm.modules[u], kUnits[u].image);
    } else {
      e = hipModuleLoad(&dm.modules[u], file.c_str());
    }
    if (e != hipSuccess) {
      dm.error = std::string("loading gfx950 code object ") + (path.empty() ? kUnits[u].name : file) +
                 ": " + hipGetErrorString(e);
      dm.status = NSR_ERR_NOT_INIT;
      return;
    }
  }
  // every kernel handle, once: a code object that lacks a listed kernel is a
  // build mismatch and fails the load (not a later launch)
  for (int k = 0; k < K_COUNT; ++k) {
    e = hipModuleGetFunction(&dm.fn[k], dm.modules[kKernels[k].unit], kKernels[k].name);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      dm.error = std::string("kernel ") + kKernels[k].name + " not in code object " + kUnits[kKernels[k].unit].name +
                 ": " + hipGetErrorString(e);
      dm.status = NSR_ERR_NOT_INIT;
      return;
    }
  }
  int lds = 0;
  hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  dm.max_lds = lds;
  int ncu = 0;
  hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  dm.n_cu = ncu > 0 ? ncu : 256;
  dm.status = NSR_OK;
}

// Module of the current device, loaded on first use.
nsr_status current_module(DeviceModule** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(NSR_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(NSR_ERR_HIP, "device index %d out of range", dev);
  DeviceModule& dm = g_dev[dev];
  std::call_once(dm.once, [&] { load_module(dm, dev); });
  if (dm.status != NSR_OK) return fail(dm.status, "%s", dm.error.c_str());
  *out = &dm;
  return NSR_OK;
}

// Launch kernel k on the current device: grid (gx, gy, gz) of `block` lanes.
nsr_status launch3(KId k, unsigned gx, unsigned gy, unsigned gz, unsigned block, unsigned shmem, nsr_stream_t stream,
                   void** params) {
  if (k < 0 || k >= K_COUNT) return fail(NSR_ERR_UNSUPPORTED, "no kernel built for this variant");
  DeviceModule* dm = nullptr;
  nsr_status st = current_module(&dm);
  if (st != NSR_OK) return st;
  if (shmem > (unsigned)dm->max_lds)
    return fail(NSR_ERR_UNSUPPORTED, "%s needs %u bytes of LDS, device allows %d", kKernels[k].name, shmem,
                dm->max_lds);
  hipError_t e =
      hipModuleLaunchKernel(dm->fn[k], gx, gy, gz, block, 1, 1, shmem, (hipStream_t)stream, params, nullptr);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // reported through nsr_status, not left sticky
    return fail(NSR_ERR_HIP, "launch %s: %s", kKernels[k].name, hipGetErrorString(e));
  }
  return NSR_OK;
}

nsr_status launch(KId k, unsigned gx, unsigned gy, unsigned block, unsigned shmem, nsr_stream_t stream,
                  void** params) {
  return launch3(k, gx, gy, 1, block, shmem, stream, params);
}

// Workgroups of kernel k (always launched with `block` lanes and `lds` bytes) that fit on one CU; cached.
int occupancy(DeviceModule* dm, KId k, unsigned block, unsigned lds) {
  int n = dm->occupancy[k].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, dm->fn[k], (int)block, lds) != hipSuccess) {
      (void)hipGetLastError();
      return 1;
    }
    n = std::max(n, 1);
    dm->occupancy[k].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Index of v in the options list, or -1.
template <size_t N>
int index_of(const int (&opts)[N], int v) {
  for (size_t i = 0; i < N; ++i)
    if (opts[i] == v) return (int)i;
  return -1;
}

template <size_t N>
KId pick(const KId (&ids)[N], int i) {
  return i >= 0 && i < (int)N ? ids[i] : K_NONE;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int dt_size(nsr_dtype d) { return d == NSR_F32 ? 4 : 2; }
bool dt_valid(nsr_dtype d) { return d == NSR_F32 || d == NSR_F16 || d == NSR_BF16; }
const char* dt_name(nsr_dtype d) { return d == NSR_F32 ? "f32" : d == NSR_F16 ? "f16" : "bf16"; }
bool act_valid(nsr_act a) { return a == NSR_ACT_NONE || a == NSR_ACT_SILU || a == NSR_ACT_GELU_ERF; }

unsigned cdiv_u(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

extern "C" {

const char* nsr_version(void) { return "nspeech-rocm 0.1.0 (gfx950)"; }

const char* nsr_last_error(void) { return g_last_error.c_str(); }

nsr_status nsr_init(const char* code_object_dir) {
  {
    std::lock_guard<std::mutex> lk(g_path_mu);
    g_code_object_path = code_object_dir ? code_object_dir : "";
  }
  DeviceModule* dm = nullptr;
  nsr_status st = current_module(&dm);
  if (st != NSR_OK) return st;
  // set up this device's fixed scratch for the entry points that allocate nothing; a failure here is
  // reported by those entry points when they are called
  int dev = 0;
  float* scratch_ptr = nullptr;
  if (hipGetDevice(&dev) == hipSuccess) (void)nsr_scratch_device_ptr(dev, &scratch_ptr);
  return NSR_OK;
}

int nsr_kernel_count(void) {
  DeviceModule* dm = nullptr;
  if (current_module(&dm) != NSR_OK) return 0;
  return K_COUNT;  // every listed kernel was resolved when the modules were loaded
}

// ------------------------------------------------------------ LayerNorm --

#define NSR_LN_FAM(p) {K_##p##_nc1, K_##p##_nc2, K_##p##_nc4, K_##p##_nc8, K_NONE, K_##p##_generic}
#define NSR_LN_FAM16(p) {K_##p##_nc1, K_##p##_nc2, K_##p##_nc4, K_##p##_nc8, K_##p##_nc16, K_##p##_generic}
// [x dtype][y dtype] (NSR_F32, NSR_F16, NSR_BF16)
static const KId kLn[3][3][6] = {
    {NSR_LN_FAM16(nsrk_ln_f32_f32), NSR_LN_FAM(nsrk_ln_f32_f16), NSR_LN_FAM(nsrk_ln_f32_bf16)},
    {NSR_LN_FAM(nsrk_ln_f16_f32), NSR_LN_FAM(nsrk_ln_f16_f16), NSR_LN_FAM(nsrk_ln_f16_bf16)},
    {NSR_LN_FAM(nsrk_ln_bf16_f32), NSR_LN_FAM(nsrk_ln_bf16_f16), NSR_LN_FAM(nsrk_ln_bf16_bf16)}};
static const KId kResLn[3][6] = {NSR_LN_FAM16(nsrk_resln_f32), NSR_LN_FAM(nsrk_resln_f16),
                                 NSR_LN_FAM(nsrk_resln_bf16)};
static const KId kResLnF16F32[6] = NSR_LN_FAM(nsrk_resln_f16f32);
#undef NSR_LN_FAM
#undef NSR_LN_FAM16

static nsr_status ln_common(const void* x, nsr_dtype xd, const void* res, nsr_dtype rd, void* h,
                            nsr_dtype hd, const void* gamma, const void* beta, nsr_dtype pd, void* y,
                            nsr_dtype yd, int64_t n_rows, int64_t n_cols, int64_t ld_x, int64_t ld_y,
                            float eps, unsigned flags, nsr_act act, bool fused, nsr_stream_t stream) {
  if (!x || !y || (fused && !res)) return fail(NSR_ERR_BAD_ARG, "layernorm: null tensor pointer");
  if (!dt_valid(xd) || !dt_valid(yd) || (fused && (!dt_valid(rd) || !dt_valid(hd))))
    return fail(NSR_ERR_BAD_ARG, "layernorm: invalid dtype");
  if (pd != NSR_F32 && pd != NSR_F16) return fail(NSR_ERR_BAD_ARG, "layernorm: params must be F32 or F16");
  if (!act_valid(act)) return fail(NSR_ERR_BAD_ARG, "layernorm: invalid activation %d", (int)act);
  if (flags & ~NSR_LN_UNIT_OFFSET) return fail(NSR_ERR_BAD_ARG, "layernorm: unknown flags 0x%x", flags);
  if (n_rows < 0 || n_cols <= 0 || n_cols > (1 << 30))
    return fail(NSR_ERR_BAD_ARG, "layernorm: bad shape rows=%lld cols=%lld", (long long)n_rows,
                (long long)n_cols);
  if (ld_x < n_cols || ld_y < n_cols) return fail(NSR_ERR_BAD_ARG, "layernorm: row stride < n_cols");
  if (!(eps >= 0.0f)) return fail(NSR_ERR_BAD_ARG, "layernorm: eps must be >= 0");
  if (n_rows == 0) return NSR_OK;

  // kernel family: [nc 1, 2, 4, 8, 16, generic]
  const KId* fam = nullptr;
  if (fused) {
    if (xd == rd && rd == hd && hd == yd) {
      fam = kResLn[xd];
    } else if (xd == NSR_F16 && rd == NSR_F32 && hd == NSR_F32 && yd == NSR_F16) {
      fam = kResLnF16F32;
    } else {
      return fail(NSR_ERR_UNSUPPORTED,
                  "residual_add_layernorm: dtype profile x=%s res=%s h=%s y=%s not built "
                  "(supported: all equal, or f16/f32/f32/f16)",
                  dt_name(xd), dt_name(rd), dt_name(hd), dt_name(yd));
    }
  } else {
    fam = kLn[xd][yd];
  }

  const bool all32 = xd == NSR_F32 && yd == NSR_F32 && (!fused || (rd == NSR_F32 && hd == NSR_F32));
  const int vec = all32 ? 4 : 8;
  bool vector_ok = (n_cols % vec == 0) && (ld_x % vec == 0) && (ld_y % vec == 0) && aligned(x, 16) &&
                   aligned(y, 16) && (!fused || aligned(res, 16)) && (!h || aligned(h, 16)) &&
                   aligned(gamma, 16) && aligned(beta, 16);
  int nc = 0;
  if (vector_ok) {
    const int64_t nchunk = n_cols / vec;
    const int opts[] = {1, 2, 4, 8, 16};
    for (int o : opts) {
      if (o == 16 && !all32) break;
      if (64 * (int64_t)o >= nchunk) {
        nc = o;
        break;
      }
    }
  }
  nsr_ln_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x;
  a.res = res;
  a.h = h;
  a.gamma = gamma;
  a.beta = beta;
  a.y = y;
  a.n_rows = n_rows;
  a.ld_x = ld_x;
  a.ld_y = ld_y;
  a.n_cols = (int32_t)n_cols;
  a.unit_offset = (flags & NSR_LN_UNIT_OFFSET) ? 1 : 0;
  a.eps = eps;
  a.inv_n = 1.0f / (float)n_cols;
  int mode = (pd == NSR_F32 ? 0 : 1) | ((int)act << 8);
  if (nc > 0 && n_cols == 64LL * nc * vec) mode |= 1 << 16;  // every chunk of every lane in the row
  void* params[] = {&a, &mode};
  if (nc > 0) {
    // Four rows (waves) per workgroup; past kLnMaxGrid workgroups each wave
    // walks rows with the grid's wave count as stride (measured best on
    // gfx950 for [24000, 1024] bf16: 4096 workgroups).
    constexpr int64_t kLnMaxGrid = 4096;
    const int64_t groups = (n_rows + 3) / 4;
    static const int kNcOpts[] = {1, 2, 4, 8, 16};
    return launch(fam[index_of(kNcOpts, nc)], (unsigned)(groups < kLnMaxGrid ? groups : kLnMaxGrid), 1,
                  256, 0, stream, params);
  }
  if (n_rows > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "layernorm: too many rows");
  return launch(fam[5], (unsigned)n_rows, 1, 256, 0, stream, params);
}

nsr_status nsr_layernorm(const void* x, nsr_dtype x_dtype, const void* gamma, const void* beta,
                         nsr_dtype param_dtype, void* y, nsr_dtype y_dtype, int64_t n_rows,
                         int64_t n_cols, int64_t ld_x, int64_t ld_y, float eps, unsigned flags,
                         nsr_act act, nsr_stream_t stream) {
  return ln_common(x, x_dtype, nullptr, x_dtype, nullptr, x_dtype, gamma, beta, param_dtype, y, y_dtype,
                   n_rows, n_cols, ld_x, ld_y, eps, flags, act, false, stream);
}

nsr_status nsr_residual_add_layernorm(const void* x, nsr_dtype x_dtype, const void* res,
                                      nsr_dtype res_dtype, void* h_out, nsr_dtype h_dtype,
                                      const void* gamma, const void* beta, nsr_dtype param_dtype,
                                      void* y, nsr_dtype y_dtype, int64_t n_rows, int64_t n_cols,
                                      float eps, unsigned flags, nsr_act act, nsr_stream_t stream) {
  return ln_common(x, x_dtype, res, res_dtype, h_out, h_dtype, gamma, beta, param_dtype, y, y_dtype,
                   n_rows, n_cols, n_cols, n_cols, eps, flags, act, true, stream);
}

// --------------------------------------------------------------- rotary --

nsr_status nsr_rope_table_f32(float* host_table, int64_t max_pos, int rotary_dim, float theta) {
  if (!host_table) return fail(NSR_ERR_BAD_ARG, "rope_table: null table");
  if (max_pos < 0 || rotary_dim <= 0 || rotary_dim % 2 != 0)
    return fail(NSR_ERR_BAD_ARG, "rope_table: bad max_pos/rotary_dim");
  const int half = rotary_dim / 2;
  // f32 arithmetic, op for op as src/moonshine/gpu_decoder.rs:328-338
  for (int i = 0; i < half; ++i) {
    const float e = (2.0f * (float)i) / (float)rotary_dim;
    const float inv_freq = 1.0f / powf(theta, e);
    for (int64_t p = 0; p < max_pos; ++p) {
      const float angle = (float)p * inv_freq;
      host_table[p * 2 * half + i] = cosf(angle);
      host_table[p * 2 * half + half + i] = sinf(angle);
    }
  }
  return NSR_OK;
}

nsr_status nsr_rotary_partial_interleaved_f32(const float* q, const float* k, float* q_out,
                                              float* k_out, int64_t B, int64_t Hq, int64_t Hk,
                                              int64_t T, int64_t Dh, int rotary_dim, float theta,
                                              int64_t pos0, const float* rope_table,
                                              int64_t table_rows, nsr_stream_t stream) {
  if (!q || !q_out) return fail(NSR_ERR_BAD_ARG, "rotary: null q/q_out");
  if (k && !k_out) return fail(NSR_ERR_BAD_ARG, "rotary: k given without k_out");
  if (B < 0 || Hq < 0 || (k && Hk < 0) || T <= 0 || Dh <= 0 || pos0 < 0)
    return fail(NSR_ERR_BAD_ARG, "rotary: bad shape");
  if (rotary_dim < 0 || rotary_dim > Dh || rotary_dim % 2 != 0)
    return fail(NSR_ERR_BAD_ARG, "rotary: rotary_dim %d must be even and <= head_dim %lld", rotary_dim,
                (long long)Dh);
  if (Dh % 4 != 0 || rotary_dim % 4 != 0)
    return fail(NSR_ERR_UNSUPPORTED, "rotary: head_dim and rotary_dim must be multiples of 4");
  if (rotary_dim / 2 > NSR_MAX_HALF_ROT) return fail(NSR_ERR_UNSUPPORTED, "rotary: rotary_dim > 256");
  if (!aligned(q, 16) || !aligned(q_out, 16) || (k && (!aligned(k, 16) || !aligned(k_out, 16))))
    return fail(NSR_ERR_BAD_ARG, "rotary: q/k/outputs must be 16-byte aligned");
  if (rope_table && (table_rows < pos0 + T || !aligned(rope_table, 8)))
    return fail(NSR_ERR_BAD_ARG, "rotary: rope table needs >= pos0+T rows and 8-byte alignment");
  if (!rope_table && !(theta > 0.0f)) return fail(NSR_ERR_BAD_ARG, "rotary: theta must be > 0");

  nsr_rope_args a;
  std::memset(&a, 0, sizeof(a));
  a.src[0] = q;
  a.dst[0] = q_out;
  a.src[1] = k ? k : q;
  a.dst[1] = k ? k_out : q_out;
  a.rows[0] = B * Hq * T;
  a.rows[1] = k ? B * Hk * T : 0;
  a.n4[0] = a.rows[0] * (Dh / 4);
  a.n4[1] = a.rows[1] * (Dh / 4);
  const int64_t total = a.n4[0] + a.n4[1];
  if (total == 0) return NSR_OK;
  if (total >= (int64_t)1 << 31) return fail(NSR_ERR_UNSUPPORTED, "rotary: tensors too large (>8 GiB)");
  a.table = rope_table;
  a.pos0 = pos0;
  a.T = (int32_t)T;
  a.dh4 = (int32_t)(Dh / 4);
  a.rot4 = rotary_dim / 4;
  a.half = rotary_dim / 2;
  // inv_freq with the reference's f32 operations (src/moonshine/decoder.rs:90-92)
  for (int i = 0; i < a.half; ++i) {
    const float e = (2.0f * (float)i) / (float)rotary_dim;
    a.inv_freq[i] = 1.0f / powf(theta, e);
  }
  void* params[] = {&a};
  return launch(rope_table ? K_nsrk_rope_table_f32 : K_nsrk_rope_compute_f32, cdiv_u(total, 256), 1, 256, 0,
                stream, params);
}

// --------------------------------------------------- decode RoPE + cache --

static nsr_status rope_cache_launch(void* q, void* k, const void* v, nsr_dtype dtype, const float* table,
                                    int64_t table_rows, void* cache_k, void* cache_v, int64_t Hq, int64_t Hk,
                                    int64_t Dh, int rot, int64_t pos, int64_t L, bool k_required,
                                    nsr_stream_t stream, const char* what) {
  if (dtype != NSR_F16 && dtype != NSR_F32) return fail(NSR_ERR_UNSUPPORTED, "%s: dtype must be F16 or F32", what);
  if (Hq < 0 || Hk < 0 || Dh <= 0 || Dh % 2 != 0 || rot < 0 || rot % 2 != 0 || rot > Dh)
    return fail(NSR_ERR_BAD_ARG, "%s: need even head_dim > 0 and even rotary_dim <= head_dim", what);
  if (pos < 0 || L <= 0 || pos >= L) return fail(NSR_ERR_BAD_ARG, "%s: pos %lld outside the cache of %lld", what,
                                                 (long long)pos, (long long)L);
  if (Hq > 0x7fff || Hk > 0x7fff || Dh > 0x7fff) return fail(NSR_ERR_UNSUPPORTED, "%s: too many heads", what);
  const uintptr_t al = dtype == NSR_F16 ? 4 : 8;
  const int half = rot / 2;
  const bool use_k = k_required && Hk > 0;  // kv_cache_append passes no k
  const bool need_q = Hq > 0 && half > 0;
  if ((need_q && (!q || !aligned(q, al))) || (use_k && (!k || !aligned(k, al) || !cache_k || !aligned(cache_k, al))))
    return fail(NSR_ERR_BAD_ARG, "%s: null or misaligned q/k/cache_k", what);
  if ((v == nullptr) != (cache_v == nullptr)) return fail(NSR_ERR_BAD_ARG, "%s: v and cache_v go together", what);
  if (v && (!aligned(v, al) || !aligned(cache_v, al))) return fail(NSR_ERR_BAD_ARG, "%s: misaligned v/cache_v", what);
  if (half > 0 && (!table || table_rows <= pos || !aligned(table, 4)))
    return fail(NSR_ERR_BAD_ARG, "%s: RoPE table needs more than pos = %lld rows", what, (long long)pos);
  nsr_rope_cache_args a;
  std::memset(&a, 0, sizeof(a));
  a.q = q;
  a.k = k;
  a.v = v;
  a.table = table;
  a.cache_k = cache_k;
  a.cache_v = cache_v;
  a.pos = pos;
  a.max_kv_len = L;
  a.Dh = (int32_t)Dh;
  a.half = half;
  a.nq = need_q ? (int32_t)(Hq * half) : 0;
  a.nk = use_k ? (int32_t)(Hk * half) : 0;
  a.nkp = use_k ? (int32_t)(Hk * (Dh - rot) / 2) : 0;
  a.nv = v ? (int32_t)(Hk * Dh / 2) : 0;
  const int64_t total = (int64_t)a.nq + a.nk + a.nkp + a.nv;
  if (total == 0) return NSR_OK;
  void* params[] = {&a};
  return launch(dtype == NSR_F16 ? K_nsrk_rope_cache_f16 : K_nsrk_rope_cache_f32, cdiv_u(total, 256), 1, 256, 0,
                stream, params);
}

nsr_status nsr_rope_qk_cache_append(void* q, void* k, const void* v, nsr_dtype dtype, const float* rope_table,
                                    int64_t table_rows, void* cache_k, void* cache_v, int64_t n_q_heads,
                                    int64_t n_kv_heads, int64_t head_dim, int rotary_dim, int64_t pos,
                                    int64_t max_kv_len, nsr_stream_t stream) {
  return rope_cache_launch(q, k, v, dtype, rope_table, table_rows, cache_k, cache_v, n_q_heads, n_kv_heads,
                           head_dim, rotary_dim, pos, max_kv_len, true, stream, "rope_qk_cache_append");
}

nsr_status nsr_kv_cache_append(const void* new_kv, void* cache, nsr_dtype dtype, int64_t n_kv_heads,
                               int64_t head_dim, int64_t max_kv_len, int64_t pos, nsr_stream_t stream) {
  if (!new_kv || !cache) return fail(NSR_ERR_BAD_ARG, "kv_cache_append: null pointer");
  return rope_cache_launch(nullptr, nullptr, new_kv, dtype, nullptr, 0, nullptr, cache, 0, n_kv_heads, head_dim, 0,
                           pos, max_kv_len, false, stream, "kv_cache_append");
}

// ------------------------------------------------------ decode attention --

namespace {

// compile-time head_dim / 4 variants of the attention kernels (d0: any head_dim)
const int kAttnHd4[] = {9, 13, 16, 32};
const KId kAttnPartial[] = {K_nsrk_attn_partial_d9, K_nsrk_attn_partial_d13, K_nsrk_attn_partial_d16,
                            K_nsrk_attn_partial_d32};
const KId kAttnHead[] = {K_nsrk_attn_head_d9, K_nsrk_attn_head_d13, K_nsrk_attn_head_d16, K_nsrk_attn_head_d32};
KId attn_kernel(const KId (&ids)[4], KId any, int64_t head_dim) {
  const int i = index_of(kAttnHd4, (int)(head_dim / 4));
  return i >= 0 ? ids[i] : any;
}

int64_t attn_wave_lds_bytes(int64_t head_dim) { return 4 * (2 * 64 * (head_dim / 4 + 1) * 2 + 64 + 256 + 64); }

void attn_fill(nsr_attn_args& a, const void* q, const void* k, const void* v, void* out, float* partial,
               int64_t kv_len, int64_t head_dim, int64_t n_kv_heads, int64_t n_q_heads, float sm_scale,
               int64_t stride_kv_head, int64_t stride_kv_seq, int64_t n_splits) {
  std::memset(&a, 0, sizeof(a));
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.out = (uint16_t*)out;
  a.partial = partial;
  a.stride_kv_head = stride_kv_head;
  a.stride_kv_seq = stride_kv_seq;
  a.kv_len = (int32_t)kv_len;
  a.n_q_heads = (int32_t)n_q_heads;
  a.n_kv_heads = (int32_t)n_kv_heads;
  a.head_dim = (int32_t)head_dim;
  a.n_splits = (int32_t)n_splits;
  a.kv_per_split = (int32_t)((kv_len + n_splits - 1) / n_splits);
  a.sm_scale = sm_scale;
}

nsr_status attn_validate(const void* q, const void* k, const void* v, void* out, int64_t kv_len, int64_t head_dim,
                         int64_t n_kv_heads, int64_t n_q_heads, float sm_scale, int64_t stride_kv_head,
                         int64_t stride_kv_seq, const char* what) {
  if (!q || !k || !v || !out) return fail(NSR_ERR_BAD_ARG, "%s: null pointer", what);
  if (kv_len < 1 || kv_len > 0x7fffffffLL || n_q_heads < 1 || n_kv_heads < 1 || n_q_heads > 65535 ||
      n_kv_heads > n_q_heads)
    return fail(NSR_ERR_BAD_ARG, "%s: bad shape kv_len=%lld n_q_heads=%lld n_kv_heads=%lld", what,
                (long long)kv_len, (long long)n_q_heads, (long long)n_kv_heads);
  if (head_dim < 4 || head_dim > 128 || head_dim % 4 != 0)
    return fail(NSR_ERR_UNSUPPORTED, "%s: head_dim=%lld must be a multiple of 4 in [4, 128]", what,
                (long long)head_dim);
  if (stride_kv_head < 0 || stride_kv_seq < head_dim || stride_kv_head % 4 != 0 || stride_kv_seq % 4 != 0)
    return fail(NSR_ERR_BAD_ARG, "%s: strides must be multiples of 4 elements, stride_kv_seq >= head_dim", what);
  if (!aligned(q, 8) || !aligned(k, 8) || !aligned(v, 8) || !aligned(out, 2))
    return fail(NSR_ERR_BAD_ARG, "%s: q, k, v need 8-byte alignment", what);
  if (!(sm_scale == sm_scale)) return fail(NSR_ERR_BAD_ARG, "%s: sm_scale is NaN", what);
  return NSR_OK;
}

}  // namespace

namespace {

// Validation shared by the split-KV entry points (partial checked by the caller).
nsr_status splitkv_validate(const void* q, const void* k, const void* v, void* out, int64_t kv_len, int64_t head_dim,
                            int64_t n_kv_heads, int64_t n_q_heads, float sm_scale, int64_t stride_kv_head,
                            int64_t stride_kv_seq, int64_t n_splits, const char* what) {
  nsr_status st = attn_validate(q, k, v, out, kv_len, head_dim, n_kv_heads, n_q_heads, sm_scale, stride_kv_head,
                                stride_kv_seq, what);
  if (st != NSR_OK) return st;
  if (n_splits < 1 || n_splits > 65535 || n_q_heads * n_splits > 0x7fffffffLL)
    return fail(NSR_ERR_BAD_ARG, "%s: n_splits=%lld out of range", what, (long long)n_splits);
  return NSR_OK;
}

// The split-KV launches (partial kernel, then reduce) over a validated call.
nsr_status splitkv_launch(const void* q, const void* k, const void* v, void* out, float* partial, int64_t kv_len,
                          int64_t head_dim, int64_t n_kv_heads, int64_t n_q_heads, float sm_scale,
                          int64_t stride_kv_head, int64_t stride_kv_seq, int64_t n_splits, nsr_stream_t stream) {
  DeviceModule* dm = nullptr;
  nsr_status st = current_module(&dm);
  if (st != NSR_OK) return st;
  nsr_attn_args a;
  attn_fill(a, q, k, v, out, partial, kv_len, head_dim, n_kv_heads, n_q_heads, sm_scale, stride_kv_head,
            stride_kv_seq, n_splits);
  void* params[] = {&a};
  st = launch(attn_kernel(kAttnPartial, K_nsrk_attn_partial_d0, head_dim), (unsigned)(n_q_heads * n_splits), 1,
              64, (unsigned)attn_wave_lds_bytes(head_dim), stream, params);
  if (st != NSR_OK) return st;
  return launch(K_nsrk_attn_reduce, (unsigned)n_q_heads, 1, 128, 0, stream, params);
}

}  // namespace

nsr_status nsr_attention_splitkv_f16(const void* q, const void* k, const void* v, void* out, float* partial,
                                     int64_t kv_len, int64_t head_dim, int64_t n_kv_heads, int64_t n_q_heads,
                                     float sm_scale, int64_t stride_kv_head, int64_t stride_kv_seq, int64_t n_splits,
                                     nsr_stream_t stream) {
  nsr_status st = splitkv_validate(q, k, v, out, kv_len, head_dim, n_kv_heads, n_q_heads, sm_scale, stride_kv_head,
                                   stride_kv_seq, n_splits, "attention_splitkv");
  if (st != NSR_OK) return st;
  if (!partial) return fail(NSR_ERR_BAD_ARG, "attention_splitkv: null partial buffer");
  return splitkv_launch(q, k, v, out, partial, kv_len, head_dim, n_kv_heads, n_q_heads, sm_scale, stride_kv_head,
                        stride_kv_seq, n_splits, stream);
}

nsr_status nsr_attention_splitkv_f16_noalloc(const void* q, const void* k, const void* v, void* out, int64_t kv_len,
                                             int64_t head_dim, int64_t n_kv_heads, int64_t n_q_heads, float sm_scale,
                                             int64_t stride_kv_head, int64_t stride_kv_seq, int64_t n_splits,
                                             nsr_stream_t stream) {
  const char* what = "attention_splitkv_noalloc";
  nsr_status st = splitkv_validate(q, k, v, out, kv_len, head_dim, n_kv_heads, n_q_heads, sm_scale, stride_kv_head,
                                   stride_kv_seq, n_splits, what);
  if (st != NSR_OK) return st;
  const int64_t need = n_q_heads * n_splits * (head_dim + 2);
  if (need > NSR_NOALLOC_SCRATCH_FLOATS)
    return fail(NSR_ERR_UNSUPPORTED,
                "%s: n_q_heads * n_splits * (head_dim + 2) = %lld floats exceeds the fixed scratch of %d floats "
                "(use nsr_attention_splitkv_f16 with a caller buffer, or fewer splits)",
                what, (long long)need, NSR_NOALLOC_SCRATCH_FLOATS);
  DeviceModule* dm = nullptr;
  st = current_module(&dm);
  if (st != NSR_OK) return st;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(NSR_ERR_HIP, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
  float* scratch_ptr = nullptr;
  e = nsr_scratch_device_ptr(dev, &scratch_ptr);
  if (e != hipSuccess || !scratch_ptr)
    return fail(NSR_ERR_HIP, "%s: resolving the fixed scratch: %s", what, hipGetErrorString(e));
  // every (head, split) slot the reduce reads is written by the partial kernel of the same call: nothing in the
  // scratch needs clearing
  return splitkv_launch(q, k, v, out, scratch_ptr, kv_len, head_dim, n_kv_heads, n_q_heads, sm_scale, stride_kv_head,
                        stride_kv_seq, n_splits, stream);
}

nsr_status nsr_attention_decode_f16(const void* q, const void* k, const void* v, void* out, int64_t kv_len,
                                    int64_t head_dim, int64_t n_kv_heads, int64_t n_q_heads, float sm_scale,
                                    int64_t stride_kv_head, int64_t stride_kv_seq, nsr_stream_t stream) {
  nsr_status st = attn_validate(q, k, v, out, kv_len, head_dim, n_kv_heads, n_q_heads, sm_scale, stride_kv_head,
                                stride_kv_seq, "attention_decode");
  if (st != NSR_OK) return st;
  DeviceModule* dm = nullptr;
  st = current_module(&dm);
  if (st != NSR_OK) return st;
  // one workgroup per query head, its waves taking every W-th chunk of 64 positions
  const int64_t per_wave = attn_wave_lds_bytes(head_dim);
  const int64_t fit = (dm->max_lds - 1024) / per_wave; /* 1 KB for the static q and merge slots */
  const int64_t W = std::max<int64_t>(1, std::min<int64_t>({8, fit, (kv_len + 63) / 64}));
  nsr_attn_args a;
  attn_fill(a, q, k, v, out, nullptr, kv_len, head_dim, n_kv_heads, n_q_heads, sm_scale, stride_kv_head,
            stride_kv_seq, 1);
  void* params[] = {&a};
  return launch(attn_kernel(kAttnHead, K_nsrk_attn_head_d0, head_dim), (unsigned)n_q_heads, 1,
                (unsigned)(64 * W), (unsigned)(W * per_wave), stream, params);
}

// -------------------------------------------------------- AdaIN + Snake --

nsr_status nsr_adain_snake_f32(const float* x, const void* gamma, const void* beta, const void* alpha,
                               nsr_dtype param_dtype, int64_t gamma_bstride, int64_t beta_bstride,
                               float* out, int64_t B, int64_t C, int64_t T, float eps,
                               nsr_stream_t stream) {
  if (!x || !gamma || !beta || !alpha || !out) return fail(NSR_ERR_BAD_ARG, "adain_snake: null pointer");
  if (param_dtype != NSR_F32 && param_dtype != NSR_F16)
    return fail(NSR_ERR_BAD_ARG, "adain_snake: params must be F32 or F16");
  if (B < 0 || C <= 0 || T <= 0 || C > 0x7fffffffLL)
    return fail(NSR_ERR_BAD_ARG, "adain_snake: bad shape B=%lld C=%lld T=%lld", (long long)B, (long long)C,
                (long long)T);
  if (gamma_bstride < 0 || beta_bstride < 0) return fail(NSR_ERR_BAD_ARG, "adain_snake: negative stride");
  if (!(eps >= 0.0f)) return fail(NSR_ERR_BAD_ARG, "adain_snake: eps must be >= 0");
  const int64_t n_rows = B * C;
  if (n_rows == 0) return NSR_OK;
  if (n_rows > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "adain_snake: too many rows");
  if (n_rows * T >= (int64_t)1 << 34) return fail(NSR_ERR_UNSUPPORTED, "adain_snake: tensor too large");

  DeviceModule* dm = nullptr;
  nsr_status st = current_module(&dm);
  if (st != NSR_OK) return st;

  nsr_adain_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x;
  a.gamma = gamma;
  a.beta = beta;
  a.alpha = alpha;
  a.out = out;
  a.n_rows = n_rows;
  a.T = T;
  a.gamma_bstride = gamma_bstride;
  a.beta_bstride = beta_bstride;
  a.C = (int32_t)C;
  a.eps = eps;
  a.inv_t = 1.0f / (float)T;
  int pdt = param_dtype == NSR_F32 ? 0 : 1;

  const bool is_aligned = aligned(x, 16) && aligned(out, 16) && (T % 4 == 0);
  KId kid = K_NONE;
  unsigned block = 0, lds = 0;
  if (is_aligned) {
    // Row kernel: BLOCK-wide slots of 16-byte chunks, NV in VGPRs + NL in LDS. The kernel masks only its
    // last four slots at the row end, so the first NV + NL - 4 slots must lie inside every row.
    const int64_t nch = T / 4;
    int nv = 0, nl = 0;
    if (nch <= 256 * 8) {
      static const KId ids[] = {K_nsrk_adain_row_b256_v1_l0, K_nsrk_adain_row_b256_v2_l0, K_nsrk_adain_row_b256_v3_l0,
                                K_nsrk_adain_row_b256_v4_l0, K_nsrk_adain_row_b256_v5_l0, K_nsrk_adain_row_b256_v6_l0,
                                K_nsrk_adain_row_b256_v7_l0, K_nsrk_adain_row_b256_v8_l0};
      block = 256;
      nv = (int)((nch + 255) / 256);
      kid = ids[nv - 1];
    } else if (nch <= 512 * 19) {
      static const int opts[] = {5, 6, 8, 10, 12, 16, 20};
      static const KId ids[] = {K_nsrk_adain_row_b512_v5_l0,  K_nsrk_adain_row_b512_v6_l0,  K_nsrk_adain_row_b512_v8_l0,
                                K_nsrk_adain_row_b512_v10_l0, K_nsrk_adain_row_b512_v12_l0, K_nsrk_adain_row_b512_v16_l0,
                                K_nsrk_adain_row_b512_v20_l0};
      block = 512;
      for (int i = 0; i < 7 && !nv; ++i)
        if (512LL * opts[i] >= nch) {
          nv = opts[i];
          kid = ids[i];
        }
    } else if (nch <= 512 * (39 + 19)) {
      // 20..58 slots: 19 in LDS, the rest in VGPRs, exactly as many as the row needs (an LDS slot costs less
      // than a VGPR slot, and a slot past the row end still costs its loads, stores and sums)
      static const KId ids[] = {
        K_nsrk_adain_row_b512_v1_l19, K_nsrk_adain_row_b512_v2_l19, K_nsrk_adain_row_b512_v3_l19,
        K_nsrk_adain_row_b512_v4_l19, K_nsrk_adain_row_b512_v5_l19, K_nsrk_adain_row_b512_v6_l19,
        K_nsrk_adain_row_b512_v7_l19, K_nsrk_adain_row_b512_v8_l19, K_nsrk_adain_row_b512_v9_l19,
        K_nsrk_adain_row_b512_v10_l19, K_nsrk_adain_row_b512_v11_l19, K_nsrk_adain_row_b512_v12_l19,
        K_nsrk_adain_row_b512_v13_l19, K_nsrk_adain_row_b512_v14_l19, K_nsrk_adain_row_b512_v15_l19,
        K_nsrk_adain_row_b512_v16_l19, K_nsrk_adain_row_b512_v17_l19, K_nsrk_adain_row_b512_v18_l19,
        K_nsrk_adain_row_b512_v19_l19, K_nsrk_adain_row_b512_v20_l19, K_nsrk_adain_row_b512_v21_l19,
        K_nsrk_adain_row_b512_v22_l19, K_nsrk_adain_row_b512_v23_l19, K_nsrk_adain_row_b512_v24_l19,
        K_nsrk_adain_row_b512_v25_l19, K_nsrk_adain_row_b512_v26_l19, K_nsrk_adain_row_b512_v27_l19,
        K_nsrk_adain_row_b512_v28_l19, K_nsrk_adain_row_b512_v29_l19, K_nsrk_adain_row_b512_v30_l19,
        K_nsrk_adain_row_b512_v31_l19, K_nsrk_adain_row_b512_v32_l19, K_nsrk_adain_row_b512_v33_l19,
        K_nsrk_adain_row_b512_v34_l19, K_nsrk_adain_row_b512_v35_l19, K_nsrk_adain_row_b512_v36_l19,
        K_nsrk_adain_row_b512_v37_l19, K_nsrk_adain_row_b512_v38_l19, K_nsrk_adain_row_b512_v39_l19};
      block = 512;
      nl = 19;
      nv = (int)((nch + 511) / 512) - nl;
      lds = (unsigned)(nl * 512 * 16);
      kid = ids[nv - 1];
      if (lds + 1024 > (unsigned)dm->max_lds) block = 0;
    }
    const int ns = nv + nl;
    if (block && (int64_t)(ns - std::min(ns, 4)) * block > nch)
      return fail(NSR_ERR_HIP, "adain_snake: internal error: row kernel slots do not fit T=%lld", (long long)T);
  } else {
    // Unaligned rows: interior chunks 1..nch-2 resident in VGPRs, edges by element.
    const int64_t need = (T + 6) / 4 - 2 > 0 ? (T + 6) / 4 - 2 : 0;
    static const int small[] = {1, 2, 3, 4, 5, 6, 8};
    static const KId small_ids[] = {K_nsrk_adain_res_b256_nv1_u, K_nsrk_adain_res_b256_nv2_u,
                                    K_nsrk_adain_res_b256_nv3_u, K_nsrk_adain_res_b256_nv4_u,
                                    K_nsrk_adain_res_b256_nv5_u, K_nsrk_adain_res_b256_nv6_u,
                                    K_nsrk_adain_res_b256_nv8_u};
    for (int i = 0; i < 7 && !block; ++i)
      if (256LL * small[i] >= need) {
        block = 256;
        kid = small_ids[i];
      }
    static const int large[] = {12, 16, 24, 32};
    static const KId large_ids[] = {K_nsrk_adain_res_b512_nv12_u, K_nsrk_adain_res_b512_nv16_u,
                                    K_nsrk_adain_res_b512_nv24_u, K_nsrk_adain_res_b512_nv32_u};
    for (int i = 0; i < 4 && !block; ++i)
      if (512LL * large[i] >= need) {
        block = 512;
        kid = large_ids[i];
      }
  }
  void* params[] = {&a, &pdt};
  if (block) {
    a.lds_chunks = (int32_t)(lds / (16u * block));
    // as many workgroups as fit on the device at once, each walking rows with the grid as stride (one per row
    // when they all fit): a row kernel that fills a CU then overlaps the next row's reads with its writes
    unsigned grid = (unsigned)n_rows;
    if (is_aligned) grid = (unsigned)std::min<int64_t>(n_rows, (int64_t)occupancy(dm, kid, block, lds) * dm->n_cu);
    return launch(kid, grid, 1, block, lds, stream, params);
  }
  // Rows past the on-chip budget: statistics over one read, then a second read to apply (persistent grid,
  // one 1024-lane workgroup per CU, no scratch).
  const bool rows16 = T % 4 == 0 && aligned(x, 16) && aligned(out, 16);
  return launch(rows16 ? K_nsrk_adain_long4 : K_nsrk_adain_long, (unsigned)std::min<int64_t>(n_rows, dm->n_cu), 1,
                1024, 0, stream, params);
}

nsr_status nsr_adain_snake_f16(const void* x, const void* gamma, const void* beta, const void* alpha,
                               nsr_dtype param_dtype, int64_t gamma_bstride, int64_t beta_bstride, void* out,
                               int64_t B, int64_t C, int64_t T, float eps, nsr_stream_t stream) {
  if (!x || !gamma || !beta || !alpha || !out) return fail(NSR_ERR_BAD_ARG, "adain_snake_f16: null pointer");
  if (param_dtype != NSR_F32 && param_dtype != NSR_F16)
    return fail(NSR_ERR_BAD_ARG, "adain_snake_f16: params must be F32 or F16");
  if (B < 0 || C <= 0 || T <= 0 || C > 0x7fffffffLL)
    return fail(NSR_ERR_BAD_ARG, "adain_snake_f16: bad shape B=%lld C=%lld T=%lld", (long long)B, (long long)C,
                (long long)T);
  if (gamma_bstride < 0 || beta_bstride < 0) return fail(NSR_ERR_BAD_ARG, "adain_snake_f16: negative stride");
  if (!(eps >= 0.0f)) return fail(NSR_ERR_BAD_ARG, "adain_snake_f16: eps must be >= 0");
  if (!aligned(x, 2) || !aligned(out, 2)) return fail(NSR_ERR_BAD_ARG, "adain_snake_f16: misaligned pointer");
  if ((((uintptr_t)x ^ (uintptr_t)out) & 15) != 0)
    return fail(NSR_ERR_BAD_ARG, "adain_snake_f16: out must have the same offset within 16 bytes as x");
  const int64_t n_rows = B * C;
  if (n_rows == 0) return NSR_OK;
  if (n_rows > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "adain_snake_f16: too many rows");
  if (T > 131072) return fail(NSR_ERR_UNSUPPORTED, "adain_snake_f16: rows longer than 131072 elements");
  // rows starting on 16 bytes (T % 8 == 0, x and out 16-byte aligned) up to T = 8192: the aligned kernel
  if (aligned(x, 16) && aligned(out, 16) && T % 8 == 0 && T <= 8 * 256 * 4) {
    static const KId ids[] = {K_nsrk_adain_f16a_b256_nv1, K_nsrk_adain_f16a_b256_nv2, K_nsrk_adain_f16a_b256_nv3,
                              K_nsrk_adain_f16a_b256_nv4};
    nsr_adain_h_args a;
    std::memset(&a, 0, sizeof(a));
    a.x = (const uint16_t*)x;
    a.gamma = gamma;
    a.beta = beta;
    a.alpha = alpha;
    a.out = (uint16_t*)out;
    a.n_rows = n_rows;
    a.T = T;
    a.gamma_bstride = gamma_bstride;
    a.beta_bstride = beta_bstride;
    a.C = (int32_t)C;
    a.eps = eps;
    a.inv_t = 1.0f / (float)T;
    int pdt = param_dtype == NSR_F32 ? 0 : 1;
    void* params[] = {&a, &pdt};
    return launch(ids[(T / 8 + 255) / 256 - 1], (unsigned)n_rows, 1, 256, 0, stream, params);
  }
  if (aligned(x, 16) && aligned(out, 16) && T % 8 == 0 && T / 8 > 512 * 19) {
    // long aligned rows (20-32 slots of 512 lanes x 8 halves): the persistent row kernel, 10 slots in LDS and
    // the rest in VGPRs, each CU's reads of its next row overlapping its writes of this one
    static const KId ids[] = {K_nsrk_adain_rowh_b512_v10_l10, K_nsrk_adain_rowh_b512_v11_l10,
                              K_nsrk_adain_rowh_b512_v12_l10, K_nsrk_adain_rowh_b512_v13_l10,
                              K_nsrk_adain_rowh_b512_v14_l10, K_nsrk_adain_rowh_b512_v15_l10,
                              K_nsrk_adain_rowh_b512_v16_l10, K_nsrk_adain_rowh_b512_v17_l10,
                              K_nsrk_adain_rowh_b512_v18_l10, K_nsrk_adain_rowh_b512_v19_l10,
                              K_nsrk_adain_rowh_b512_v20_l10, K_nsrk_adain_rowh_b512_v21_l10,
                              K_nsrk_adain_rowh_b512_v22_l10};
    const int64_t slots = (T / 8 + 511) / 512; /* 20..32 (T <= 131072) */
    const unsigned lds = 10u * 512u * 16u;
    DeviceModule* dm = nullptr;
    nsr_status st = current_module(&dm);
    if (st != NSR_OK) return st;
    if (slots <= 32 && lds + 1024 <= (unsigned)dm->max_lds) {
      const KId kid = ids[slots - 20];
      nsr_adain_h_args a;
      std::memset(&a, 0, sizeof(a));
      a.x = (const uint16_t*)x;
      a.gamma = gamma;
      a.beta = beta;
      a.alpha = alpha;
      a.out = (uint16_t*)out;
      a.n_rows = n_rows;
      a.T = T;
      a.gamma_bstride = gamma_bstride;
      a.beta_bstride = beta_bstride;
      a.C = (int32_t)C;
      a.eps = eps;
      a.inv_t = 1.0f / (float)T;
      int pdt = param_dtype == NSR_F32 ? 0 : 1;
      void* params[] = {&a, &pdt};
      const unsigned grid = (unsigned)std::min<int64_t>(n_rows, (int64_t)occupancy(dm, kid, 512, lds) * dm->n_cu);
      return launch(kid, grid, 1, 512, lds, stream, params);
    }
  }
  // interior 16-byte chunks of a row, at the worst offset (7 elements into its first chunk)
  const int64_t need = (T + 14) / 8 - 2;
  unsigned block = 0;
  KId kid = K_NONE;
  static const int small[] = {1, 2, 3, 4, 6, 8};
  static const KId small_ids[] = {K_nsrk_adain_f16_b256_nv1, K_nsrk_adain_f16_b256_nv2, K_nsrk_adain_f16_b256_nv3,
                                  K_nsrk_adain_f16_b256_nv4, K_nsrk_adain_f16_b256_nv6, K_nsrk_adain_f16_b256_nv8};
  for (int i = 0; i < 6 && !block; ++i)
    if (256LL * small[i] >= need) {
      block = 256;
      kid = small_ids[i];
    }
  static const int large[] = {6, 8, 12, 16, 20, 24, 28, 32};
  static const KId large_ids[] = {K_nsrk_adain_f16_b512_nv6,  K_nsrk_adain_f16_b512_nv8,  K_nsrk_adain_f16_b512_nv12,
                                  K_nsrk_adain_f16_b512_nv16, K_nsrk_adain_f16_b512_nv20, K_nsrk_adain_f16_b512_nv24,
                                  K_nsrk_adain_f16_b512_nv28, K_nsrk_adain_f16_b512_nv32};
  for (int i = 0; i < 8 && !block; ++i)
    if (512LL * large[i] >= need) {
      block = 512;
      kid = large_ids[i];
    }
  if (!block) return fail(NSR_ERR_UNSUPPORTED, "adain_snake_f16: rows longer than 131072 elements");
  nsr_adain_h_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = (const uint16_t*)x;
  a.gamma = gamma;
  a.beta = beta;
  a.alpha = alpha;
  a.out = (uint16_t*)out;
  a.n_rows = n_rows;
  a.T = T;
  a.gamma_bstride = gamma_bstride;
  a.beta_bstride = beta_bstride;
  a.C = (int32_t)C;
  a.eps = eps;
  a.inv_t = 1.0f / (float)T;
  int pdt = param_dtype == NSR_F32 ? 0 : 1;
  void* params[] = {&a, &pdt};
  return launch(kid, (unsigned)n_rows, 1, block,
                0, stream, params);
}

// --------------------------------------------------------------- Q8_0 --

nsr_status nsr_q8_0_embed_gather(const void* blocks, int64_t vocab, int64_t d, const void* ids,
                                 nsr_index_dtype id_dtype, int64_t n_ids, float* out, nsr_act act,
                                 int32_t* err_flag, nsr_stream_t stream) {
  if (!blocks || !ids || !out) return fail(NSR_ERR_BAD_ARG, "q8_0_embed_gather: null pointer");
  if (vocab <= 0 || d <= 0 || d % 32 != 0 || n_ids < 0)
    return fail(NSR_ERR_BAD_ARG, "q8_0_embed_gather: need vocab > 0, d a positive multiple of 32, n_ids >= 0");
  if (id_dtype != NSR_IDX_U32 && id_dtype != NSR_IDX_I64)
    return fail(NSR_ERR_BAD_ARG, "q8_0_embed_gather: invalid id dtype");
  if (!act_valid(act)) return fail(NSR_ERR_BAD_ARG, "q8_0_embed_gather: invalid activation");
  if (!aligned(blocks, 2) || !aligned(out, 16) || !aligned(ids, id_dtype == NSR_IDX_U32 ? 4 : 8))
    return fail(NSR_ERR_BAD_ARG, "q8_0_embed_gather: misaligned pointer (blocks 2 B, out 16 B, ids)");
  if (d / 32 * 34 > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "q8_0_embed_gather: row too long");
  if (n_ids == 0) return NSR_OK;
  const int64_t total4 = n_ids * (d / 4);
  if (total4 >= (int64_t)1 << 32 || (total4 + 255) / 256 > 0x7fffffffLL)
    return fail(NSR_ERR_UNSUPPORTED, "q8_0_embed_gather: output too large");
  nsr_q8_args a;
  std::memset(&a, 0, sizeof(a));
  a.blocks = (const uint8_t*)blocks;
  a.ids = ids;
  a.out = out;
  a.err_flag = err_flag;
  a.vocab = vocab;
  a.n_ids = n_ids;
  a.total4 = total4;
  a.d4 = (int32_t)(d / 4);
  a.row_bytes = (int32_t)(d / 32 * 34);
  a.act = (int32_t)act;
  a.ids_i64 = id_dtype == NSR_IDX_I64;
  static const KId kGather[2][3] = {
      {K_nsrk_q8_0_gather_none_u32, K_nsrk_q8_0_gather_silu_u32, K_nsrk_q8_0_gather_gelu_u32},
      {K_nsrk_q8_0_gather_none_i64, K_nsrk_q8_0_gather_silu_i64, K_nsrk_q8_0_gather_gelu_i64}};
  // Rows of 64 .. 256 float4 (d 256 .. 1024): each id on whole waves (gw of them), ids per workgroup so
  // it has at most 4 waves. Shorter rows: ids packed densely, whole ids per 256-lane workgroup. Longer:
  // one lane per float4 over a flat grid.
  unsigned block = 256;
  if (a.d4 >= 64 && a.d4 <= 256) {
    a.gw = (a.d4 + 63) / 64;
    a.ipw = 4 / a.gw;
    block = 64u * (unsigned)(a.gw * a.ipw);
  } else {
    a.ipw = a.d4 < 64 ? 256 / a.d4 : 0;
  }
  const int64_t groups = a.ipw ? (n_ids + a.ipw - 1) / a.ipw : cdiv_u(total4, 256);
  if (groups > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "q8_0_embed_gather: too many ids");
  void* params[] = {&a};
  return launch(kGather[id_dtype == NSR_IDX_I64][act], (unsigned)groups, 1, block, 0, stream, params);
}

// ---------------------------------------------------------- elementwise --

enum EwOp { kEwSilu, kEwGelu, kEwGlu, kEwAdd };
// [op][dtype][vector, scalar]
static const KId kEw[4][3][2] = {
    {{K_nsrk_silu_f32_v, K_nsrk_silu_f32_s}, {K_nsrk_silu_f16_v, K_nsrk_silu_f16_s},
     {K_nsrk_silu_bf16_v, K_nsrk_silu_bf16_s}},
    {{K_nsrk_gelu_f32_v, K_nsrk_gelu_f32_s}, {K_nsrk_gelu_f16_v, K_nsrk_gelu_f16_s},
     {K_nsrk_gelu_bf16_v, K_nsrk_gelu_bf16_s}},
    {{K_nsrk_glu_f32_v, K_nsrk_glu_f32_s}, {K_nsrk_glu_f16_v, K_nsrk_glu_f16_s}, {K_nsrk_glu_bf16_v, K_nsrk_glu_bf16_s}},
    {{K_nsrk_add_f32_v, K_nsrk_add_f32_s}, {K_nsrk_add_f16_v, K_nsrk_add_f16_s}, {K_nsrk_add_bf16_v, K_nsrk_add_bf16_s}}};

static nsr_status ew_launch(EwOp opi, nsr_dtype dtype, nsr_ew_args& a, bool vec_ok, nsr_stream_t stream) {
  static const char* const kOpName[] = {"silu", "gelu", "glu", "add"};
  const char* op = kOpName[opi];
  const int vec = 16 / dt_size(dtype);
  int64_t first = 0;
  if (vec_ok) {
    const int64_t chunks = a.n / vec;
    if (chunks > 0) {
      if ((chunks + 255) / 256 > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "%s: too large", op);
      void* p[] = {&a};
      nsr_status st = launch(kEw[opi][dtype][0], cdiv_u(chunks, 256), 1,
                             256, 0, stream, p);
      if (st != NSR_OK) return st;
    }
    first = chunks * vec;
  }
  const int64_t rest = a.n - first;
  if (rest > 0) {
    if ((rest + 255) / 256 > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "%s: too large", op);
    void* p[] = {&a, &first};
    return launch(kEw[opi][dtype][1], cdiv_u(rest, 256), 1, 256, 0, stream,
                  p);
  }
  return NSR_OK;
}

// f32 combine: out = lrelu?(((a + b) + c) * scale)
static nsr_status combine_launch(const float* a, const float* b, const float* c, float* out, int64_t n, bool scale,
                                 float s, bool lrelu, float slope, nsr_stream_t stream, const char* what) {
  if (!a || !out) return fail(NSR_ERR_BAD_ARG, "%s: null pointer", what);
  if (n < 0) return fail(NSR_ERR_BAD_ARG, "%s: n < 0", what);
  if (!aligned(a, 4) || !aligned(out, 4) || (b && !aligned(b, 4)) || (c && !aligned(c, 4)))
    return fail(NSR_ERR_BAD_ARG, "%s: misaligned pointer", what);
  if (n == 0) return NSR_OK;
  nsr_combine_args g;
  std::memset(&g, 0, sizeof(g));
  g.a = a;
  g.b = b;
  g.c = c;
  g.out = out;
  g.n = n;
  g.scale = s;
  g.slope = slope;
  g.flags = (scale ? 1 : 0) | (lrelu ? 2 : 0);
  const bool vec = aligned(a, 16) && aligned(out, 16) && (!b || aligned(b, 16)) && (!c || aligned(c, 16));
  int64_t first = 0;
  if (vec && n / 4 > 0) {
    if ((n / 4 + 255) / 256 > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "%s: too large", what);
    void* p[] = {&g};
    nsr_status st = launch(K_nsrk_combine_f32_v, cdiv_u(n / 4, 256), 1, 256, 0, stream, p);
    if (st != NSR_OK) return st;
    first = n / 4 * 4;
  }
  if (n > first) {
    if ((n - first + 255) / 256 > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "%s: too large", what);
    void* p[] = {&g, &first};
    return launch(K_nsrk_combine_f32_s, cdiv_u(n - first, 256), 1, 256, 0, stream, p);
  }
  return NSR_OK;
}

nsr_status nsr_scale_f32(const float* x, float* out, int64_t n, float s, nsr_stream_t stream) {
  return combine_launch(x, nullptr, nullptr, out, n, true, s, false, 0.f, stream, "scale_f32");
}

nsr_status nsr_leaky_relu_f32(const float* x, float* out, int64_t n, float slope, nsr_stream_t stream) {
  return combine_launch(x, nullptr, nullptr, out, n, false, 1.f, true, slope, stream, "leaky_relu_f32");
}

nsr_status nsr_resblock_average_f32(const float* r0, const float* r1, const float* r2, float* out, int64_t n,
                                    int leaky_relu, float slope, nsr_stream_t stream) {
  if (!r1 || !r2) return fail(NSR_ERR_BAD_ARG, "resblock_average_f32: null pointer");
  // the reference's elementwise_scale_third_f32 multiplies by the f32 nearest 1/3
  return combine_launch(r0, r1, r2, out, n, true, (float)0.3333333333333333, leaky_relu != 0, slope, stream,
                        "resblock_average_f32");
}

nsr_status nsr_snake(const void* x, nsr_dtype dtype, const void* alpha, nsr_dtype alpha_dtype, void* out,
                     int64_t n_elements, int64_t channels, int64_t seq_len, nsr_stream_t stream) {
  if (!x || !alpha || !out) return fail(NSR_ERR_BAD_ARG, "snake: null pointer");
  if (dtype != NSR_F32 && dtype != NSR_F16) return fail(NSR_ERR_BAD_ARG, "snake: x must be F32 or F16");
  if (alpha_dtype != NSR_F32 && alpha_dtype != NSR_F16) return fail(NSR_ERR_BAD_ARG, "snake: alpha must be F32 or F16");
  if (n_elements < 0 || channels <= 0 || channels > 0x7fffffffLL || seq_len <= 0 || n_elements % seq_len != 0)
    return fail(NSR_ERR_BAD_ARG, "snake: need channels > 0, seq_len > 0 dividing n_elements");
  const int esz = dtype == NSR_F32 ? 4 : 2;
  if (!aligned(x, esz) || !aligned(out, esz) || !aligned(alpha, alpha_dtype == NSR_F32 ? 4 : 2))
    return fail(NSR_ERR_BAD_ARG, "snake: misaligned pointer");
  if (n_elements == 0) return NSR_OK;
  nsr_snake_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x;
  a.alpha = alpha;
  a.out = out;
  a.T = seq_len;
  a.chunks = (seq_len + 1023) / 1024;
  a.C = (int32_t)channels;
  a.pdt = alpha_dtype == NSR_F32 ? 0 : 1;
  const int64_t blocks = n_elements / seq_len * a.chunks;
  if (blocks > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "snake: too large");
  void* params[] = {&a};
  return launch(dtype == NSR_F32 ? K_nsrk_snake_f32 : K_nsrk_snake_f16, (unsigned)blocks, 1, 256, 0, stream, params);
}

// ------------------------------------------------------------------ iSTFT --

nsr_status nsr_istft_f32(const float* x, float* out, int64_t n_frames, int64_t out_len, int n_fft, int hop,
                         nsr_stream_t stream) {
  if (!x || !out) return fail(NSR_ERR_BAD_ARG, "istft: null pointer");
  if (n_frames < 1 || hop < 1 || n_fft < 2 || n_fft % hop != 0)
    return fail(NSR_ERR_BAD_ARG, "istft: need n_frames >= 1 and hop dividing n_fft");
  if (n_frames * (n_fft + 2) >= (1LL << 31))  // x holds 2 (n_fft / 2 + 1) rows of n_frames
    return fail(NSR_ERR_UNSUPPORTED, "istft: input larger than 2^31 elements");
  if (n_fft != 16 && n_fft != 20 && n_fft != 32)
    return fail(NSR_ERR_UNSUPPORTED, "istft: n_fft %d not built (16, 20, 32)", n_fft);
  if (out_len < 0 || out_len > (n_frames - 1) * (int64_t)hop)
    return fail(NSR_ERR_BAD_ARG, "istft: out_len must be in [0, (n_frames - 1) * hop]");
  if (!aligned(x, 4) || !aligned(out, 4)) return fail(NSR_ERR_BAD_ARG, "istft: misaligned pointer");
  if (out_len == 0) return NSR_OK;
  nsr_istft_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x;
  a.out = out;
  a.n_frames = n_frames;
  a.out_len = out_len;
  a.n_fft = n_fft;
  a.hop = hop;
  // 64 frames per workgroup (the kernel's NSR_ISTFT_FG); neighbours overlap by n_fft / hop - 1 frames
  const int64_t FG = 64, R = n_fft / hop, step = FG - (R - 1);
  a.frames_per_group = (int32_t)FG;
  const int64_t groups = n_frames <= FG ? 1 : 1 + (n_frames - FG + step - 1) / step;
  if (groups > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "istft: too many frames");
  void* params[] = {&a};
  const KId kid = n_fft == 16 ? K_nsrk_istft_f32_n16 : n_fft == 20 ? K_nsrk_istft_f32_n20 : K_nsrk_istft_f32_n32;
  return launch(kid, (unsigned)groups, 1, 256, 0, stream, params);
}

nsr_status nsr_activation(const void* x, void* y, nsr_dtype dtype, int64_t n, nsr_act act,
                          nsr_stream_t stream) {
  if (!x || !y) return fail(NSR_ERR_BAD_ARG, "activation: null pointer");
  if (!dt_valid(dtype) || n < 0) return fail(NSR_ERR_BAD_ARG, "activation: bad dtype or n");
  if (act != NSR_ACT_SILU && act != NSR_ACT_GELU_ERF)
    return fail(NSR_ERR_BAD_ARG, "activation: act must be SILU or GELU_ERF");
  if (n == 0) return NSR_OK;
  nsr_ew_args a;
  std::memset(&a, 0, sizeof(a));
  a.a = x;
  a.out = y;
  a.n = n;
  a.act = (int32_t)act;
  return ew_launch(act == NSR_ACT_SILU ? kEwSilu : kEwGelu, dtype, a, aligned(x, 16) && aligned(y, 16), stream);
}

nsr_status nsr_glu_silu(const void* fc1, void* out, nsr_dtype dtype, int64_t n, nsr_stream_t stream) {
  if (!fc1 || !out) return fail(NSR_ERR_BAD_ARG, "glu_silu: null pointer");
  if (!dt_valid(dtype) || n < 0) return fail(NSR_ERR_BAD_ARG, "glu_silu: bad dtype or n");
  if (n == 0) return NSR_OK;
  nsr_ew_args a;
  std::memset(&a, 0, sizeof(a));
  a.a = fc1;
  a.out = out;
  a.n = n;
  const bool ok = aligned(fc1, 16) && aligned(out, 16) && ((n * dt_size(dtype)) % 16 == 0);
  return ew_launch(kEwGlu, dtype, a, ok, stream);
}

nsr_status nsr_residual_add(const void* x, const void* res, void* out, nsr_dtype dtype, int64_t n,
                            nsr_stream_t stream) {
  if (!x || !res || !out) return fail(NSR_ERR_BAD_ARG, "residual_add: null pointer");
  if (!dt_valid(dtype) || n < 0) return fail(NSR_ERR_BAD_ARG, "residual_add: bad dtype or n");
  if (n == 0) return NSR_OK;
  nsr_ew_args a;
  std::memset(&a, 0, sizeof(a));
  a.a = x;
  a.b = res;
  a.out = out;
  a.n = n;
  return ew_launch(kEwAdd, dtype, a, aligned(x, 16) && aligned(res, 16) && aligned(out, 16), stream);
}

}  // extern "C"

// ----------------------------------------------------------- Q8 GEMV --

namespace {

enum GemvMode { kGemvPlain = 0, kGemvGlu = 1, kGemvResLn = 2 };

// Workgroup size for t4 tiles: about one 16-byte chunk (4 rows) per lane,
// between 256 and 1024 lanes (measured on gfx950: K = 640 -> 256,
// K = 2560 -> 1024).
int t4_block(int64_t K) {
  const int64_t chunks = K / 4;
  return chunks <= 256 ? 256 : chunks <= 512 ? 512 : 1024;
}

nsr_status gemv_launch(GemvMode mode, bool t4, const void* x, nsr_dtype xd, const uint32_t* qs,
                       const uint16_t* scales, const float* bias, void* out, nsr_dtype od, const float* residual,
                       float* out_f32, const void* ln_w, nsr_dtype wd, int64_t K, int64_t N, float eps,
                       nsr_stream_t stream, const char* what) {
  if (!x || !qs || !scales || !out || (mode == kGemvResLn && (!residual || !out_f32 || !ln_w)))
    return fail(NSR_ERR_BAD_ARG, "%s: null pointer", what);
  if ((xd != NSR_F16 && xd != NSR_F32) || (od != NSR_F16 && od != NSR_F32))
    return fail(xd == NSR_BF16 || od == NSR_BF16 ? NSR_ERR_UNSUPPORTED : NSR_ERR_BAD_ARG,
                "%s: x and output dtypes must be F16 or F32", what);
  if (mode == kGemvResLn && wd != NSR_F16 && wd != NSR_F32)
    return fail(NSR_ERR_BAD_ARG, "%s: ln_weight dtype must be F16 or F32", what);
  if (K < 0 || N < 0 || K > (1LL << 30) || N > (1LL << 28))
    return fail(NSR_ERR_BAD_ARG, "%s: bad shape K=%lld N=%lld", what, (long long)K, (long long)N);
  if (K % 32 != 0) return fail(NSR_ERR_BAD_ARG, "%s: K=%lld must be a multiple of 32", what, (long long)K);
  if (N % 16 != 0) return fail(NSR_ERR_BAD_ARG, "%s: N=%lld must be a multiple of 16", what, (long long)N);
  if (!aligned(qs, 16) || !aligned(scales, 16))
    return fail(NSR_ERR_BAD_ARG, "%s: qs and scales need 16-byte alignment", what);
  // t4 kernels read x 4 elements at a time
  const uintptr_t xa = t4 ? 4 * dt_size(xd) : dt_size(xd);
  if (!aligned(x, xa) || !aligned(out, dt_size(od)) || (bias && !aligned(bias, 4)) ||
      (residual && !aligned(residual, 4)) || (out_f32 && !aligned(out_f32, 4)) ||
      (ln_w && !aligned(ln_w, dt_size(wd))))
    return fail(NSR_ERR_BAD_ARG, "%s: misaligned pointer", what);
  if (!(eps >= 0.0f)) return fail(NSR_ERR_BAD_ARG, "%s: eps must be >= 0", what);
  if (N == 0) return NSR_OK;
  if (K == 0) return fail(NSR_ERR_BAD_ARG, "%s: K must be > 0", what);

  const int64_t NW = mode == kGemvGlu ? 2 * N : N;
  nsr_gemv_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x;
  a.qs = qs;
  a.scales = scales;
  a.bias = bias;
  a.out = out;
  a.residual = residual;
  a.out_f32 = out_f32;
  a.K = (int32_t)K;
  a.NW = (int32_t)NW;
  a.N = (int32_t)N;
  void* params[] = {&a};
  // x and output dtypes are F32 (0) or F16 (1); the resadd+LN projection writes f32 h, indexed by x only
  const int xi = xd == NSR_F16, oi = od == NSR_F16;
  KId kid;
  unsigned groups, block;
  if (t4) {
    // [mode][x][out][block 256, 512, 1024]
    static const KId ids[3][2][2][3] = {
        {{{K_nsrk_gemv_q8t4_f32_f32_b256, K_nsrk_gemv_q8t4_f32_f32_b512, K_nsrk_gemv_q8t4_f32_f32_b1024},
          {K_nsrk_gemv_q8t4_f32_f16_b256, K_nsrk_gemv_q8t4_f32_f16_b512, K_nsrk_gemv_q8t4_f32_f16_b1024}},
         {{K_nsrk_gemv_q8t4_f16_f32_b256, K_nsrk_gemv_q8t4_f16_f32_b512, K_nsrk_gemv_q8t4_f16_f32_b1024},
          {K_nsrk_gemv_q8t4_f16_f16_b256, K_nsrk_gemv_q8t4_f16_f16_b512, K_nsrk_gemv_q8t4_f16_f16_b1024}}},
        {{{K_nsrk_gemv_q8t4_glu_f32_f32_b256, K_nsrk_gemv_q8t4_glu_f32_f32_b512, K_nsrk_gemv_q8t4_glu_f32_f32_b1024},
          {K_nsrk_gemv_q8t4_glu_f32_f16_b256, K_nsrk_gemv_q8t4_glu_f32_f16_b512, K_nsrk_gemv_q8t4_glu_f32_f16_b1024}},
         {{K_nsrk_gemv_q8t4_glu_f16_f32_b256, K_nsrk_gemv_q8t4_glu_f16_f32_b512, K_nsrk_gemv_q8t4_glu_f16_f32_b1024},
          {K_nsrk_gemv_q8t4_glu_f16_f16_b256, K_nsrk_gemv_q8t4_glu_f16_f16_b512, K_nsrk_gemv_q8t4_glu_f16_f16_b1024}}},
        {{{K_nsrk_gemv_q8t4_h_f32_b256, K_nsrk_gemv_q8t4_h_f32_b512, K_nsrk_gemv_q8t4_h_f32_b1024},
          {K_nsrk_gemv_q8t4_h_f32_b256, K_nsrk_gemv_q8t4_h_f32_b512, K_nsrk_gemv_q8t4_h_f32_b1024}},
         {{K_nsrk_gemv_q8t4_h_f16_b256, K_nsrk_gemv_q8t4_h_f16_b512, K_nsrk_gemv_q8t4_h_f16_b1024},
          {K_nsrk_gemv_q8t4_h_f16_b256, K_nsrk_gemv_q8t4_h_f16_b512, K_nsrk_gemv_q8t4_h_f16_b1024}}}};
    block = (unsigned)t4_block(K);
    kid = ids[mode][xi][oi][block == 256 ? 0 : block == 512 ? 1 : 2];
    groups = (unsigned)(NW / 4);
  } else {
    // [mode][x][out]
    static const KId ids[3][2][2] = {
        {{K_nsrk_gemv_q8_f32_f32, K_nsrk_gemv_q8_f32_f16}, {K_nsrk_gemv_q8_f16_f32, K_nsrk_gemv_q8_f16_f16}},
        {{K_nsrk_gemv_q8_glu_f32_f32, K_nsrk_gemv_q8_glu_f32_f16},
         {K_nsrk_gemv_q8_glu_f16_f32, K_nsrk_gemv_q8_glu_f16_f16}},
        {{K_nsrk_gemv_q8_h_f32, K_nsrk_gemv_q8_h_f32}, {K_nsrk_gemv_q8_h_f16, K_nsrk_gemv_q8_h_f16}}};
    block = 256;
    kid = ids[mode][xi][oi];
    // Tile map (kernels/gemv_q8.hip): line groups (16 tiles of one 128-byte line on one XCD) unless that leaves
    // an XCD with more tiles than both the balanced share and its 32 CUs; then contiguous runs. Measured on
    // MI355X: fc2 (80 tiles) reads 1.03x its bytes on line groups against 2.38x on runs, in the same time; fc1 + GLU
    // (320 tiles) 1.20x on runs at 8.1 us against 1.0x on line groups at 9.3 us (3 against 2 groups per XCD).
    const int64_t n_tiles = mode == kGemvGlu ? N / 8 : NW / 8;
    const int64_t per_xcd_groups = ((n_tiles + 15) / 16 + 7) / 8;
    const bool lg = 16 * per_xcd_groups <= std::max<int64_t>((n_tiles + 7) / 8, 32);
    a.n_tiles = (int32_t)n_tiles;
    a.line_groups = lg ? 1 : 0;
    groups = (unsigned)(lg ? 8 * 16 * per_xcd_groups : n_tiles);
  }
  nsr_status st = launch(kid, groups, 1, block, 0, stream, params);
  if (st != NSR_OK || mode != kGemvResLn) return st;
  // LayerNorm of the dim columns of h, weight only (one row)
  return ln_common(out_f32, NSR_F32, nullptr, NSR_F32, nullptr, NSR_F32, ln_w, nullptr, wd, out, od, 1, N, N, N, eps,
                   0, NSR_ACT_NONE, false, stream);
}

}  // namespace

extern "C" {

nsr_status nsr_gemv_q8(const void* x, nsr_dtype x_dtype, const uint32_t* qs, const uint16_t* scales,
                       const float* bias, void* out, nsr_dtype out_dtype, int64_t K, int64_t N,
                       nsr_stream_t stream) {
  return gemv_launch(kGemvPlain, false, x, x_dtype, qs, scales, bias, out, out_dtype, nullptr, nullptr, nullptr,
                     NSR_F32, K, N, 0.0f, stream, "gemv_q8");
}

nsr_status nsr_gemv_q8_bias_glu(const void* x, nsr_dtype x_dtype, const uint32_t* qs, const uint16_t* scales,
                                const float* bias, void* out, nsr_dtype out_dtype, int64_t K, int64_t N,
                                nsr_stream_t stream) {
  return gemv_launch(kGemvGlu, false, x, x_dtype, qs, scales, bias, out, out_dtype, nullptr, nullptr, nullptr,
                     NSR_F32, K, N, 0.0f, stream, "gemv_q8_bias_glu");
}

nsr_status nsr_gemv_q8_resadd_ln(const void* x, nsr_dtype x_dtype, const uint32_t* qs, const uint16_t* scales,
                                 const float* residual, float* out_f32, const void* ln_weight, nsr_dtype w_dtype,
                                 void* norm, nsr_dtype norm_dtype, int64_t K, int64_t dim, float eps,
                                 nsr_stream_t stream) {
  return gemv_launch(kGemvResLn, false, x, x_dtype, qs, scales, nullptr, norm, norm_dtype, residual, out_f32,
                     ln_weight, w_dtype, K, dim, eps, stream, "gemv_q8_resadd_ln");
}

nsr_status nsr_q8_pack_t4(const uint32_t* qs, const uint16_t* scales, int64_t K, int64_t NW, int glu,
                          uint32_t* t4_qs, uint16_t* t4_scales, nsr_stream_t stream) {
  if (!qs || !scales || !t4_qs || !t4_scales) return fail(NSR_ERR_BAD_ARG, "q8_pack_t4: null pointer");
  if (K <= 0 || NW <= 0 || K % 32 != 0 || NW % 16 != 0 || (glu && NW % 32 != 0) || K > (1LL << 30) ||
      NW > (1LL << 28) || K * NW > (1LL << 40))
    return fail(NSR_ERR_BAD_ARG, "q8_pack_t4: bad shape K=%lld NW=%lld (K %% 32 == 0, NW %% 16 == 0%s)",
                (long long)K, (long long)NW, glu ? ", NW % 32 == 0 for GLU" : "");
  if (!aligned(qs, 4) || !aligned(scales, 2) || !aligned(t4_qs, 16) || !aligned(t4_scales, 16))
    return fail(NSR_ERR_BAD_ARG, "q8_pack_t4: misaligned pointer (outputs need 16 bytes)");
  nsr_q8_pack_args a;
  std::memset(&a, 0, sizeof(a));
  a.qs = (const uint8_t*)qs;
  a.scales = scales;
  a.tq = t4_qs;
  a.ts = t4_scales;
  a.K = (int32_t)K;
  a.NW = (int32_t)NW;
  a.N = glu ? (int32_t)(NW / 2) : 0;
  const int64_t total = (NW / 4) * K + (NW / 4) * (K / 32);
  void* params[] = {&a};
  return launch(K_nsrk_gemv_q8t4_pack, cdiv_u(total, 256), 1, 256, 0, stream, params);
}

static nsr_status q8_0_convert(const void* blocks, int64_t N, int64_t K, int t4, int glu, uint32_t* qs,
                               uint16_t* scales, nsr_stream_t stream, const char* what) {
  if (!blocks || !qs || !scales) return fail(NSR_ERR_BAD_ARG, "%s: null pointer", what);
  if (N <= 0 || K <= 0 || K % 32 != 0 || N % 16 != 0 || (glu && N % 32 != 0) || K > (1LL << 30) ||
      N > (1LL << 28) || N * K > (1LL << 40))
    return fail(NSR_ERR_BAD_ARG, "%s: bad shape N=%lld K=%lld (K %% 32 == 0, N %% 16 == 0%s)", what, (long long)N,
                (long long)K, glu ? ", N % 32 == 0 for GLU" : "");
  if (!aligned(blocks, 2) || !aligned(qs, 16) || !aligned(scales, 16))
    return fail(NSR_ERR_BAD_ARG, "%s: misaligned pointer (blocks 2 bytes, outputs 16 bytes)", what);
  nsr_q8_0_conv_args a;
  std::memset(&a, 0, sizeof(a));
  a.blocks = (const uint8_t*)blocks;
  a.qs = qs;
  a.scales = scales;
  a.N = (int32_t)N;
  a.K = (int32_t)K;
  a.t4 = t4;
  a.glu_n = glu ? (int32_t)(N / 2) : 0;
  const int64_t total = (N / 4) * K;  // one thread per output word; the first of each block moves its scales
  void* params[] = {&a};
  return launch(K_nsrk_gemv_q8_from_q8_0, cdiv_u(total, 256), 1, 256, 0, stream, params);
}

nsr_status nsr_q8_0_to_gemv_q8(const void* blocks, int64_t N, int64_t K, uint32_t* qs, uint16_t* scales,
                               nsr_stream_t stream) {
  return q8_0_convert(blocks, N, K, 0, 0, qs, scales, stream, "q8_0_to_gemv_q8");
}

nsr_status nsr_q8_0_to_t4(const void* blocks, int64_t N, int64_t K, int glu, uint32_t* t4_qs, uint16_t* t4_scales,
                          nsr_stream_t stream) {
  return q8_0_convert(blocks, N, K, 1, glu ? 1 : 0, t4_qs, t4_scales, stream, "q8_0_to_t4");
}

nsr_status nsr_gemv_q8_t4(const void* x, nsr_dtype x_dtype, const uint32_t* t4_qs, const uint16_t* t4_scales,
                          const float* bias, void* out, nsr_dtype out_dtype, int64_t K, int64_t N,
                          nsr_stream_t stream) {
  return gemv_launch(kGemvPlain, true, x, x_dtype, t4_qs, t4_scales, bias, out, out_dtype, nullptr, nullptr, nullptr,
                     NSR_F32, K, N, 0.0f, stream, "gemv_q8_t4");
}

nsr_status nsr_gemv_q8_t4_bias_glu(const void* x, nsr_dtype x_dtype, const uint32_t* t4_qs,
                                   const uint16_t* t4_scales, const float* bias, void* out, nsr_dtype out_dtype,
                                   int64_t K, int64_t N, nsr_stream_t stream) {
  return gemv_launch(kGemvGlu, true, x, x_dtype, t4_qs, t4_scales, bias, out, out_dtype, nullptr, nullptr, nullptr,
                     NSR_F32, K, N, 0.0f, stream, "gemv_q8_t4_bias_glu");
}

nsr_status nsr_gemv_q8_t4_resadd_ln(const void* x, nsr_dtype x_dtype, const uint32_t* t4_qs,
                                    const uint16_t* t4_scales, const float* residual, float* out_f32,
                                    const void* ln_weight, nsr_dtype w_dtype, void* norm, nsr_dtype norm_dtype,
                                    int64_t K, int64_t dim, float eps, nsr_stream_t stream) {
  return gemv_launch(kGemvResLn, true, x, x_dtype, t4_qs, t4_scales, nullptr, norm, norm_dtype, residual, out_f32,
                     ln_weight, w_dtype, K, dim, eps, stream, "gemv_q8_t4_resadd_ln");
}

}  // extern "C"

// ------------------------------------------------------- Kokoro conv1d --

namespace {

constexpr int kCvTT = 64, kCvCO = 128, kCvCI = 128, kCvS = kCvCI + 8, kCvMaxTL = 128;
constexpr int64_t kConvMaxSlabBytes = 0xffffffffLL;  // a buffer descriptor's byte range

nsr_status conv_validate(const float* x, const void* w, uintptr_t w_align, float* out, int64_t B, int64_t C_in,
                         int64_t C_out, int64_t T_in, int64_t K, int64_t padding, int64_t dilation, int64_t* T_out,
                         const char* what) {
  if (!x || !w || !out) return fail(NSR_ERR_BAD_ARG, "%s: null pointer", what);
  if (B < 0 || C_in <= 0 || C_out <= 0 || T_in < 0 || K <= 0 || padding < 0 || dilation <= 0 || B > 65535 ||
      C_out > 65535LL * kCvCO || C_in > (1 << 20) || K > 4096 || dilation > (1 << 20) || padding > (1 << 24) ||
      T_in >= (1LL << 23))
    return fail(NSR_ERR_BAD_ARG, "%s: bad shape B=%lld C_in=%lld C_out=%lld T=%lld K=%lld pad=%lld dil=%lld", what,
                (long long)B, (long long)C_in, (long long)C_out, (long long)T_in, (long long)K, (long long)padding,
                (long long)dilation);
  if (C_in % 16 != 0) return fail(NSR_ERR_UNSUPPORTED, "%s: C_in=%lld must be a multiple of 16", what, (long long)C_in);
  *T_out = T_in + 2 * padding - dilation * (K - 1);
  // rows of 128 channels are addressed with 32-bit byte offsets
  if (*T_out >= (1LL << 23)) return fail(NSR_ERR_BAD_ARG, "%s: T_out=%lld too long", what, (long long)*T_out);
  if (*T_out <= 0 && T_in > 0)
    return fail(NSR_ERR_BAD_ARG, "%s: empty output (T_in + 2 padding < dilation (K - 1) + 1)", what);
  // each batch's input, output and residual rows are addressed through one buffer descriptor, whose byte
  // range (and every offset in it) is 32-bit
  if (4 * C_in * T_in > kConvMaxSlabBytes || 4 * C_out * std::max<int64_t>(*T_out, 0) > kConvMaxSlabBytes)
    return fail(NSR_ERR_UNSUPPORTED, "%s: one batch's rows (C_in %lld x T_in %lld, C_out %lld x T_out %lld f32) "
                "exceed the %lld bytes a buffer descriptor addresses", what, (long long)C_in, (long long)T_in,
                (long long)C_out, (long long)*T_out, (long long)kConvMaxSlabBytes);
  if (!aligned(x, 4) || !aligned(out, 4) || !aligned(w, w_align))
    return fail(NSR_ERR_BAD_ARG, "%s: misaligned pointer (weights need %u bytes)", what, (unsigned)w_align);
  return NSR_OK;
}

#define NSR_CONV_NU(p) {{K_##p##_nu3, K_##p##_nu4}, {K_##p##_nu3_st, K_##p##_nu4_st}}
// [fused][residual][row statistics][nu 3, 4]
const KId kConvRw[2][2][2][2] = {
    {NSR_CONV_NU(nsrk_conv1d_rw_f16x2), NSR_CONV_NU(nsrk_conv1d_rw_res_f16x2)},
    {NSR_CONV_NU(nsrk_conv1d_rw_adain_snake_f16x2), NSR_CONV_NU(nsrk_conv1d_rw_adain_snake_res_f16x2)}};
const KId kConvPc[2][2][2][2] = {
    {NSR_CONV_NU(nsrk_conv1d_pc_f16x2), NSR_CONV_NU(nsrk_conv1d_pc_res_f16x2)},
    {NSR_CONV_NU(nsrk_conv1d_pc_adain_snake_f16x2), NSR_CONV_NU(nsrk_conv1d_pc_adain_snake_res_f16x2)}};
#undef NSR_CONV_NU
// [fused][np 9, 12, 16]
const KId kConvNp[2][3] = {
    {K_nsrk_conv1d_f16x2_np9, K_nsrk_conv1d_f16x2_np12, K_nsrk_conv1d_f16x2_np16},
    {K_nsrk_conv1d_adain_snake_f16x2_np9, K_nsrk_conv1d_adain_snake_f16x2_np12, K_nsrk_conv1d_adain_snake_f16x2_np16}};

nsr_status conv_launch(bool fused, nsr_conv_args& a, nsr_stream_t stream, const char* what, bool* emitted = nullptr) {
  DeviceModule* dm = nullptr;
  nsr_status st = current_module(&dm);
  if (st != NSR_OK) return st;
  const int64_t TL = kCvTT + (int64_t)(a.K - 1) * a.dilation;
  const int64_t lds = (2 * TL + kCvCO) * kCvS * 2; /* y hi, y lo, one tap's weights */
  if (TL > kCvMaxTL || lds > dm->max_lds)
    return fail(NSR_ERR_UNSUPPORTED, "%s: (K - 1) * dilation = %lld needs %lld bytes of LDS, device allows %d", what,
                (long long)((a.K - 1) * (int64_t)a.dilation), (long long)lds, dm->max_lds);
  // 16-byte epilogue stores when every output (and residual) row starts 16-byte aligned
  a.pad_ = (a.T_out % 4 == 0 && aligned(a.out, 16) && (!a.residual || aligned(a.residual, 16))) ? 1 : 0;
  void* params[] = {&a};
  // persistent workgroups: as many as fit at once (two per CU when the LDS allows), each walking tiles
  const int64_t tiles = (int64_t)cdiv_u(a.T_out, kCvTT) * cdiv_u(a.C_out, kCvCO) * a.B;
  if (tiles > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "%s: too many tiles", what);
  const int np = TL <= 72 ? 9 : TL <= 96 ? 12 : 16;  // register pairs per lane: 8 TL <= 64 np
  // K <= 3 with one channel block each way and 16-byte aligned rows: every weight resident in LDS,
  // one 512-lane workgroup per CU (producer and consumer waves)
  const int64_t lds_rw = ((int64_t)a.K * kCvCO + 2 * TL) * kCvS * 2;
  const int64_t win = TL + ((-(int64_t)a.padding) & 3);  // staged window from a 16-byte aligned column
  if (a.C_in <= kCvCI && a.C_out <= kCvCO && a.K <= 3 && win <= 128 && lds_rw <= dm->max_lds && (a.pad_ & 1) &&
      a.T_in > 0 && a.T_in % 4 == 0 && aligned(a.x, 16)) {
    const int64_t groups = std::min<int64_t>(tiles, (int64_t)dm->n_cu);
    if (emitted) *emitted = a.row_part != nullptr;
    return launch(kConvRw[fused][a.residual != nullptr][a.row_part != nullptr][win <= 96 ? 0 : 1], (unsigned)groups,
                  1, 512, (unsigned)lds_rw, stream, params);
  }
  // any K, C_in in chunks and C_out in blocks of 128, 16-byte aligned rows: weights streamed one tap ahead
  // through two LDS slots, one 512-lane workgroup per CU (producer and consumer waves)
  const int64_t lds_pc = (2 * TL + 2 * kCvCO) * kCvS * 2 + 4 * (int64_t)a.C_out; /* + the bias as f32 */
  if (win <= 128 && lds_pc <= dm->max_lds && (a.pad_ & 1) && a.T_in > 0 && a.T_in % 4 == 0 && aligned(a.x, 16)) {
    const int64_t groups = std::min<int64_t>(tiles, (int64_t)dm->n_cu);
    if (emitted) *emitted = a.row_part != nullptr;
    return launch(kConvPc[fused][a.residual != nullptr][a.row_part != nullptr][win <= 96 ? 0 : 1], (unsigned)groups,
                  1, 512, (unsigned)lds_pc, stream, params);
  }
  // the plain np 9 kernel fits two workgroups per CU in registers; the others one (no row statistics: the
  // caller takes them from the output)
  if (emitted) *emitted = false;
  const int per_cu = (!fused && np == 9 && 2 * lds <= dm->max_lds) ? 2 : 1;
  const int64_t groups = std::min<int64_t>(tiles, (int64_t)per_cu * dm->n_cu);
  return launch(kConvNp[fused][np == 9 ? 0 : np == 12 ? 1 : 2], (unsigned)groups, 1, 256, (unsigned)lds, stream,
                params);
}

}  // namespace

extern "C" {

nsr_status nsr_conv1d_pack_f16(const void* w, int64_t C_out, int64_t C_in, int64_t K, void* w_packed,
                               nsr_stream_t stream) {
  if (!w || !w_packed) return fail(NSR_ERR_BAD_ARG, "conv1d_pack_f16: null pointer");
  if (C_out <= 0 || C_in <= 0 || K <= 0 || C_out * C_in * K > (1LL << 34))
    return fail(NSR_ERR_BAD_ARG, "conv1d_pack_f16: bad shape");
  if (!aligned(w, 2) || !aligned(w_packed, 16)) return fail(NSR_ERR_BAD_ARG, "conv1d_pack_f16: misaligned pointer");
  nsr_conv_pack_args a;
  a.w = (const uint16_t*)w;
  a.wp = (uint16_t*)w_packed;
  a.C_out = C_out;
  a.C_in = C_in;
  a.K = K;
  void* params[] = {&a};
  return launch(K_nsrk_conv1d_pack, cdiv_u(C_out * C_in * K, 256), 1, 256, 0, stream, params);
}

// Records of the pre-split conv: B x ceil(C_in / 128) x (T_in + 2 padding) records of 512 bytes, then the
// weights in MFMA fragment order, ceil(C_out / 128) x 4 x K x ceil(C_in / 128) x 8 KB.
static int64_t conv_records_only_bytes(int64_t B, int64_t C_in, int64_t Tp) {
  return (B * ((C_in + 127) / 128) * Tp * 512 + 255) / 256 * 256;
}
static int64_t conv_records_bytes(int64_t B, int64_t C_in, int64_t C_out, int64_t K, int64_t Tp) {
  return conv_records_only_bytes(B, C_in, Tp) + (C_out + 127) / 128 * 4 * K * ((C_in + 127) / 128) * 8192;
}

// The record path: a bandwidth-bound pass writes the input's records (AdaIN + Snake when fused, the f16
// hi / lo split, [t][ci] order) and the weights in fragment order into the caller's workspace, then the MFMA
// kernel reads them with no per-element VALU work. Taken when `records` is given and the rows qualify; else
// the one-launch kernels.
static constexpr int kCvTW = 128;
static constexpr unsigned kCvRingLds = 256 * 528 + 56 * 512;  // record ring + the output staging rows after it
static nsr_status conv_records(bool fused, nsr_conv_args& a, char* records, nsr_stream_t stream, const char* what,
                               bool* emitted = nullptr) {
  DeviceModule* dm = nullptr;
  nsr_status st = current_module(&dm);
  if (st != NSR_OK) return st;
  const int64_t D = (int64_t)(a.K - 1) * a.dilation;
  const int64_t TLe = kCvTW + D + (D & 1);
  const bool rows16 = a.T_out % 4 == 0 && aligned(a.out, 16) && (!a.residual || aligned(a.residual, 16));
  // TLe <= 184 leaves 72 ring slots outside a window, which with the 56 rows after the ring stage a 128-row tile.
  // Below K = 7 the records pass (x read, records written) costs more than the one-launch kernels lose to
  // their per-element work (measured on MI355X at [8, 128, 115200]: K = 3 about 540 us against 370 us).
  if (!records || a.K < 7 || !rows16 || TLe > 184 || a.C_out % 2 != 0 || kCvRingLds > dm->max_lds || a.T_in <= 0)
    return conv_launch(fused, a, stream, what, emitted);
  const int64_t Tp = (int64_t)a.T_in + 2 * a.padding;
  const int64_t n_ch = (a.C_in + 127) / 128, n_co = (a.C_out + 127) / 128;
  // records pass blocks: 64 input columns each, from column -64 * ceil(padding / 64) (the leading padding)
  const int64_t rec_blocks = (int64_t)a.B * n_ch * (((int64_t)a.T_in + a.padding + 63) / 64 + (a.padding + 63) / 64);
  const int64_t w_blocks = n_co * 4 * a.K * n_ch * 2;  // fragment weights: 16 bytes per lane, 8 KB = 2 blocks
  const int64_t blocks = (rec_blocks + w_blocks + 7) / 8 * 8;
  if (blocks > 0x7fffffffLL || Tp * 512 > 0xffffffffLL) return conv_launch(fused, a, stream, what, emitted);
  uint8_t* xs = (uint8_t*)records;
  uint8_t* wf = (uint8_t*)records + conv_records_only_bytes(a.B, a.C_in, Tp);
  void* pp[] = {&a, &xs, &wf};
  st = launch(fused ? K_nsrk_conv_presplit_adain_snake : K_nsrk_conv_presplit, (unsigned)blocks, 1, 256, 0, stream, pp);
  if (st != NSR_OK) return st;
  a.pad_ = 1;
  const int64_t tiles = (int64_t)cdiv_u(a.T_out, kCvTW) * n_co * a.B;
  if (tiles > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "%s: too many tiles", what);
  const bool stats = a.row_part != nullptr;
  if (emitted) *emitted = stats;
  // statistics: the _st32 kernels when every 32-column block is whole (T_out % 32 == 0: no column masks)
  static const KId ids[2][3] = {{K_nsrk_conv1d_pr_f16x2, K_nsrk_conv1d_pr_f16x2_st, K_nsrk_conv1d_pr_f16x2_st32},
                                {K_nsrk_conv1d_pr_res_f16x2, K_nsrk_conv1d_pr_res_f16x2_st,
                                 K_nsrk_conv1d_pr_res_f16x2_st32}};
  // one workgroup per CU, a multiple of 8 (the kernel's XCD split) when there are enough tiles
  int64_t grid = std::min<int64_t>(tiles, dm->n_cu);
  if (grid >= 8) grid = grid / 8 * 8;
  const int kv = stats ? (a.T_out % 32 == 0 ? 2 : 1) : 0;
  return launch(ids[a.residual != nullptr][kv], (unsigned)grid, 1, 512, kCvRingLds, stream, pp);
}

// Launch a conv and leave the per-(b, co) statistics of its output in row_stats ([B*C_out][2]: mean,
// 1 / sqrt(var + eps)): the aligned-row kernels emit per-32-column (mean, M2) blocks from their epilogue into
// `part` (the caller's workspace, [B*C_out][ceil(T_out / 32)][2] f32) and a merge kernel combines them; the
// fallback kernel's output is re-read by the row statistics kernel instead.
static nsr_status conv_launch_stats(bool fused, nsr_conv_args& a, float eps, float* row_stats, float* part,
                                    char* records, nsr_stream_t stream, const char* what) {
  const int64_t rows = (int64_t)a.B * a.C_out, nblk = ((int64_t)a.T_out + 31) / 32;
  if (rows > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "%s: too many rows", what);
  a.row_part = part;
  bool emitted = false;
  nsr_status st = conv_records(fused, a, records, stream, what, &emitted);
  if (st == NSR_OK && emitted) {
    nsr_rowstats_args m;
    std::memset(&m, 0, sizeof(m));
    m.part = part;
    m.stats = row_stats;
    m.nblk = (int32_t)nblk;
    m.T_out = a.T_out;
    m.eps = eps;
    void* pm[] = {&m};
    st = launch(K_nsrk_conv_rowstats_merge, (unsigned)rows, 1, 256, 0, stream, pm);
  } else if (st == NSR_OK) {
    nsr_adain_args s;
    std::memset(&s, 0, sizeof(s));
    s.x = a.out;
    s.stats = row_stats;
    s.n_rows = rows;
    s.T = a.T_out;
    s.C = a.C_out;
    s.eps = eps;
    s.inv_t = 1.0f / (float)a.T_out;
    void* ps[] = {&s};
    const bool rows16 = a.T_out % 4 == 0 && aligned(a.out, 16);
    st = launch(rows16 ? K_nsrk_adain_stats4 : K_nsrk_adain_stats, (unsigned)rows, 1, 1024, 0, stream, ps);
  }
  a.row_part = nullptr;
  return st;
}

// Workspace parts of the conv entry points, each at a 256-byte aligned offset in the order of the flags.
static int64_t ws_round(int64_t b) { return (b + 255) / 256 * 256; }

static void conv_ws_layout(int64_t B, int64_t C_in, int64_t C_out, int64_t T_out, int64_t K, int64_t Tp,
                           unsigned parts, int64_t off[4], int64_t* total) {
  int64_t o = 0;
  const int64_t sz[4] = {ws_round(C_out * C_in * K * 2), ws_round(B * C_in * 2 * 4),
                         ws_round(B * C_out * ((T_out + 31) / 32) * 2 * 4), ws_round(conv_records_bytes(B, C_in, C_out, K, Tp))};
  for (int i = 0; i < 4; ++i) {
    off[i] = -1;
    if (parts & (1u << i)) {
      off[i] = o;
      o += sz[i];
    }
  }
  *total = o;
}

// Check the caller's workspace and return the address of each requested part. The records part is
// optional: present (ptr[3]) when the workspace also covers it, after the required parts.
static nsr_status conv_ws_parts(void* workspace, int64_t workspace_bytes, int64_t B, int64_t C_in, int64_t C_out,
                                int64_t T_out, int64_t K, int64_t Tp, unsigned parts, char* ptr[4],
                                const char* what) {
  int64_t off[4], need = 0;
  conv_ws_layout(B, C_in, C_out, std::max<int64_t>(T_out, 0), K, Tp, parts, off, &need);
  if (need > 0 && (!workspace || !aligned(workspace, 256) || workspace_bytes < need))
    return fail(NSR_ERR_BAD_ARG, "%s: needs a 256-byte aligned workspace of %lld bytes (nsr_conv1d_workspace_bytes)",
                what, (long long)need);
  for (int i = 0; i < 4; ++i) ptr[i] = off[i] >= 0 ? (char*)workspace + off[i] : nullptr;
  int64_t roff[4], rneed = 0;
  conv_ws_layout(B, C_in, C_out, std::max<int64_t>(T_out, 0), K, Tp, parts | NSR_WS_RECORDS, roff, &rneed);
  if (workspace && aligned(workspace, 256) && workspace_bytes >= rneed) ptr[3] = (char*)workspace + roff[3];
  return NSR_OK;
}

static nsr_status conv_packed_impl(const float* x, const void* w_packed, const void* bias, const float* residual,
                                   float* out, int64_t B, int64_t C_in, int64_t C_out, int64_t T_in, int64_t K,
                                   int64_t padding, int64_t dilation, char* records, nsr_stream_t stream) {
  int64_t T_out = 0;
  nsr_status st = conv_validate(x, w_packed, 16, out, B, C_in, C_out, T_in, K, padding, dilation, &T_out,
                                "conv1d_f16w_packed");
  if (st != NSR_OK) return st;
  if ((bias && !aligned(bias, 2)) || (residual && !aligned(residual, 4)))
    return fail(NSR_ERR_BAD_ARG, "conv1d_f16w_packed: misaligned bias or residual");
  if (B == 0 || T_out <= 0) return NSR_OK;  // T_in == 0 with T_out > 0: output = bias (+ residual)
  nsr_conv_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x;
  a.w = (const uint16_t*)w_packed;
  a.bias = (const uint16_t*)bias;
  a.residual = residual;
  a.out = out;
  a.B = (int32_t)B;
  a.C_in = (int32_t)C_in;
  a.C_out = (int32_t)C_out;
  a.T_in = (int32_t)T_in;
  a.T_out = (int32_t)T_out;
  a.K = (int32_t)K;
  a.padding = (int32_t)padding;
  a.dilation = (int32_t)dilation;
  return conv_records(false, a, records, stream, "conv1d_f16w_packed");
}

nsr_status nsr_conv1d_f16w_packed(const float* x, const void* w_packed, const void* bias, const float* residual,
                                  float* out, int64_t B, int64_t C_in, int64_t C_out, int64_t T_in, int64_t K,
                                  int64_t padding, int64_t dilation, nsr_stream_t stream) {
  return conv_packed_impl(x, w_packed, bias, residual, out, B, C_in, C_out, T_in, K, padding, dilation, nullptr,
                          stream);
}

nsr_status nsr_conv1d_f32io(const float* x, const void* w, const void* bias, float* out, int64_t B, int64_t C_in,
                            int64_t C_out, int64_t T_in, int64_t K, int64_t stride, int64_t padding,
                            int64_t dilation, void* workspace, int64_t workspace_bytes, nsr_stream_t stream) {
  if (stride != 1) return fail(NSR_ERR_UNSUPPORTED, "conv1d_f32io: stride %lld (only stride 1 is built)",
                               (long long)stride);
  int64_t T_out = 0;
  nsr_status st = conv_validate(x, w, 2, out, B, C_in, C_out, T_in, K, padding, dilation, &T_out, "conv1d_f32io");
  if (st != NSR_OK) return st;
  if (bias && !aligned(bias, 2)) return fail(NSR_ERR_BAD_ARG, "conv1d_f32io: misaligned bias");
  char* part[4];
  st = conv_ws_parts(workspace, workspace_bytes, B, C_in, C_out, T_out, K, T_in + 2 * padding, NSR_WS_PACKED_WEIGHTS,
                     part, "conv1d_f32io");
  if (st != NSR_OK) return st;
  if (B == 0 || T_out <= 0) return NSR_OK;
  // pack the weights into the caller's workspace, then convolve
  st = nsr_conv1d_pack_f16(w, C_out, C_in, K, part[0], stream);
  if (st != NSR_OK) return st;
  return conv_packed_impl(x, part[0], bias, nullptr, out, B, C_in, C_out, T_in, K, padding, dilation, part[3],
                          stream);
}

static nsr_status adain_conv_impl(const float* x, const float* x_stats, const void* gamma, const void* beta,
                                  const void* alpha, nsr_dtype param_dtype, int64_t gamma_bstride,
                                  int64_t beta_bstride, const void* w_packed, const void* bias, const float* residual,
                                  float* out, float* out_stats, int64_t B, int64_t C_in, int64_t C_out, int64_t T,
                                  int64_t K, int64_t padding, int64_t dilation, float eps, void* workspace,
                                  int64_t workspace_bytes, nsr_stream_t stream, const char* what) {
  if (!gamma || !beta || !alpha) return fail(NSR_ERR_BAD_ARG, "%s: null parameter pointer", what);
  if (param_dtype != NSR_F32 && param_dtype != NSR_F16) return fail(NSR_ERR_BAD_ARG, "%s: params must be F32 or F16", what);
  if (gamma_bstride < 0 || beta_bstride < 0) return fail(NSR_ERR_BAD_ARG, "%s: negative batch stride", what);
  if (!(eps >= 0.0f)) return fail(NSR_ERR_BAD_ARG, "%s: eps must be >= 0", what);
  if ((x_stats && !aligned(x_stats, 8)) || (out_stats && !aligned(out_stats, 8)))
    return fail(NSR_ERR_BAD_ARG, "%s: row statistics need 8-byte alignment", what);
  int64_t T_out = 0;
  nsr_status st = conv_validate(x, w_packed, 16, out, B, C_in, C_out, T, K, padding, dilation, &T_out, what);
  if (st != NSR_OK) return st;
  if ((bias && !aligned(bias, 2)) || (residual && !aligned(residual, 4)))
    return fail(NSR_ERR_BAD_ARG, "%s: misaligned bias or residual", what);
  const unsigned parts = (x_stats ? 0u : NSR_WS_IN_STATS) | (out_stats ? NSR_WS_OUT_STATS : 0u);
  char* part[4];
  st = conv_ws_parts(workspace, workspace_bytes, B, C_in, C_out, T_out, K, T + 2 * padding, parts, part, what);
  if (st != NSR_OK) return st;
  if (B == 0 || T_out <= 0) return NSR_OK;
  if (T == 0) return fail(NSR_ERR_BAD_ARG, "%s: T == 0 (an empty row has no statistics)", what);
  // per-(b, ci) mean and 1/sqrt(var + eps) of x: the caller's, or computed into the workspace
  float* stats = nullptr;
  if (!x_stats) {
    stats = (float*)part[1];
    nsr_adain_args s;
    std::memset(&s, 0, sizeof(s));
    s.x = x;
    s.stats = stats;
    s.n_rows = B * C_in;
    s.T = T;
    s.C = (int32_t)C_in;
    s.eps = eps;
    s.inv_t = 1.0f / (float)T;
    void* p1[] = {&s};
    const bool rows16 = T % 4 == 0 && aligned(x, 16);
    st = launch(rows16 ? K_nsrk_adain_stats4 : K_nsrk_adain_stats, (unsigned)(B * C_in), 1, 1024, 0, stream, p1);
  }
  if (st == NSR_OK) {
    nsr_conv_args a;
    std::memset(&a, 0, sizeof(a));
    a.x = x;
    a.w = (const uint16_t*)w_packed;
    a.bias = (const uint16_t*)bias;
    a.residual = residual;
    a.out = out;
    a.stats = x_stats ? x_stats : stats;
    a.gamma = gamma;
    a.beta = beta;
    a.alpha = alpha;
    a.gamma_bstride = gamma_bstride;
    a.beta_bstride = beta_bstride;
    a.B = (int32_t)B;
    a.C_in = (int32_t)C_in;
    a.C_out = (int32_t)C_out;
    a.T_in = (int32_t)T;
    a.T_out = (int32_t)T_out;
    a.K = (int32_t)K;
    a.padding = (int32_t)padding;
    a.dilation = (int32_t)dilation;
    a.pdt = param_dtype == NSR_F32 ? 0 : 1;
    st = out_stats ? conv_launch_stats(true, a, eps, out_stats, (float*)part[2], part[3], stream, what)
                   : conv_records(true, a, part[3], stream, what);
  }
  return st;
}

nsr_status nsr_adain_snake_conv1d_f32(const float* x, const void* gamma, const void* beta, const void* alpha,
                                      nsr_dtype param_dtype, int64_t gamma_bstride, int64_t beta_bstride,
                                      const void* w_packed, const void* bias, const float* residual, float* out,
                                      int64_t B, int64_t C_in, int64_t C_out, int64_t T, int64_t K, int64_t padding,
                                      int64_t dilation, float eps, void* workspace, int64_t workspace_bytes,
                                      nsr_stream_t stream) {
  return adain_conv_impl(x, nullptr, gamma, beta, alpha, param_dtype, gamma_bstride, beta_bstride, w_packed, bias,
                         residual, out, nullptr, B, C_in, C_out, T, K, padding, dilation, eps, workspace,
                         workspace_bytes, stream, "adain_snake_conv1d");
}

nsr_status nsr_adain_snake_conv1d_chain_f32(const float* x, const float* x_stats, const void* gamma,
                                            const void* beta, const void* alpha, nsr_dtype param_dtype,
                                            int64_t gamma_bstride, int64_t beta_bstride, const void* w_packed,
                                            const void* bias, const float* residual, float* out, float* out_stats,
                                            int64_t B, int64_t C_in, int64_t C_out, int64_t T, int64_t K,
                                            int64_t padding, int64_t dilation, float eps, void* workspace,
                                            int64_t workspace_bytes, nsr_stream_t stream) {
  return adain_conv_impl(x, x_stats, gamma, beta, alpha, param_dtype, gamma_bstride, beta_bstride, w_packed, bias,
                         residual, out, out_stats, B, C_in, C_out, T, K, padding, dilation, eps, workspace,
                         workspace_bytes, stream, "adain_snake_conv1d_chain");
}

nsr_status nsr_conv1d_f16w_packed_stats(const float* x, const void* w_packed, const void* bias,
                                        const float* residual, float* out, float* out_stats, int64_t B, int64_t C_in,
                                        int64_t C_out, int64_t T_in, int64_t K, int64_t padding, int64_t dilation,
                                        float eps, void* workspace, int64_t workspace_bytes, nsr_stream_t stream) {
  const char* what = "conv1d_f16w_packed_stats";
  int64_t T_out = 0;
  nsr_status st = conv_validate(x, w_packed, 16, out, B, C_in, C_out, T_in, K, padding, dilation, &T_out, what);
  if (st != NSR_OK) return st;
  if (!out_stats || !aligned(out_stats, 8)) return fail(NSR_ERR_BAD_ARG, "%s: null or misaligned out_stats", what);
  if ((bias && !aligned(bias, 2)) || (residual && !aligned(residual, 4)))
    return fail(NSR_ERR_BAD_ARG, "%s: misaligned bias or residual", what);
  if (!(eps >= 0.0f)) return fail(NSR_ERR_BAD_ARG, "%s: eps must be >= 0", what);
  char* part[4];
  st = conv_ws_parts(workspace, workspace_bytes, B, C_in, C_out, T_out, K, T_in + 2 * padding, NSR_WS_OUT_STATS, part,
                     what);
  if (st != NSR_OK) return st;
  if (B == 0 || T_out <= 0) return NSR_OK;
  if (T_in == 0) return fail(NSR_ERR_BAD_ARG, "%s: T_in == 0", what);
  nsr_conv_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x;
  a.w = (const uint16_t*)w_packed;
  a.bias = (const uint16_t*)bias;
  a.residual = residual;
  a.out = out;
  a.B = (int32_t)B;
  a.C_in = (int32_t)C_in;
  a.C_out = (int32_t)C_out;
  a.T_in = (int32_t)T_in;
  a.T_out = (int32_t)T_out;
  a.K = (int32_t)K;
  a.padding = (int32_t)padding;
  a.dilation = (int32_t)dilation;
  return conv_launch_stats(false, a, eps, out_stats, (float*)part[2], part[3], stream, what);
}

nsr_status nsr_conv1d_workspace_bytes(int64_t B, int64_t C_in, int64_t C_out, int64_t T_in, int64_t K,
                                      int64_t padding, int64_t dilation, unsigned parts, int64_t* bytes) {
  if (!bytes) return fail(NSR_ERR_BAD_ARG, "conv1d_workspace_bytes: null result pointer");
  *bytes = 0;
  if (parts & ~(unsigned)(NSR_WS_PACKED_WEIGHTS | NSR_WS_IN_STATS | NSR_WS_OUT_STATS | NSR_WS_RECORDS))
    return fail(NSR_ERR_BAD_ARG, "conv1d_workspace_bytes: unknown parts 0x%x", parts);
  if (B < 0 || C_in <= 0 || C_out <= 0 || T_in < 0 || K <= 0 || padding < 0 || dilation <= 0 || B > 65535 ||
      C_in > (1 << 20) || C_out > (1 << 24) || K > 4096 || T_in >= (1LL << 23) || padding > (1 << 24) ||
      dilation > (1 << 20))
    return fail(NSR_ERR_BAD_ARG, "conv1d_workspace_bytes: bad shape");
  const int64_t T_out = std::max<int64_t>(0, T_in + 2 * padding - dilation * (K - 1));
  int64_t off[4];
  conv_ws_layout(B, C_in, C_out, T_out, K, T_in + 2 * padding, parts, off, bytes);
  return NSR_OK;
}


}  // extern "C"

// ------------------------------------------------------ measurement floors --

extern "C" {

nsr_status nsr_calib_empty(nsr_stream_t stream) {
  nsr_calib_args a;
  std::memset(&a, 0, sizeof(a));
  void* params[] = {&a};
  return launch(K_nsrk_calib_empty, 1, 1, 256, 0, stream, params);
}

nsr_status nsr_calib_copy(const void* src, void* dst, int64_t bytes, int form, int groups_per_cu,
                          nsr_stream_t stream) {
  if (!src || !dst) return fail(NSR_ERR_BAD_ARG, "calib_copy: null pointer");
  if (bytes < 0 || bytes % 16 != 0 || !aligned(src, 16) || !aligned(dst, 16))
    return fail(NSR_ERR_BAD_ARG, "calib_copy: bytes must be a multiple of 16 and pointers 16-byte aligned");
  if (form < 0 || form > 2 || groups_per_cu < 0 || groups_per_cu > 64)
    return fail(NSR_ERR_BAD_ARG, "calib_copy: form must be 0, 1 or 2 and groups_per_cu in [0, 64]");
  if (bytes == 0) return NSR_OK;
  const int64_t n4 = bytes / 16;
  if ((n4 + 255) / 256 > 0x7fffffffLL) return fail(NSR_ERR_UNSUPPORTED, "calib_copy: too large");
  DeviceModule* dm = nullptr;
  nsr_status st = current_module(&dm);
  if (st != NSR_OK) return st;
  nsr_calib_args a;
  a.src = (const float*)src;
  a.dst = (float*)dst;
  a.n4 = n4;
  void* params[] = {&a};
  if (form == 0) return launch(K_nsrk_calib_copy_flat, cdiv_u(n4, 256), 1, 256, 0, stream, params);
  const int64_t tile = 256 * (form == 1 ? 4 : 8);
  const int64_t groups = std::min<int64_t>((int64_t)(groups_per_cu ? groups_per_cu : 8) * dm->n_cu, (n4 + tile - 1) / tile);
  return launch(form == 1 ? K_nsrk_calib_copy_p4 : K_nsrk_calib_copy_p8, (unsigned)groups, 1, 256, 0, stream, params);
}

nsr_status nsr_calib_copy_rows(const void* src, void* dst, int64_t n_rows, int64_t row_bytes, nsr_stream_t stream) {
  if (!src || !dst) return fail(NSR_ERR_BAD_ARG, "calib_copy_rows: null pointer");
  if (n_rows < 0 || row_bytes <= 0 || row_bytes % 16 != 0 || row_bytes >= ((int64_t)1 << 31) ||
      !aligned(src, 16) || !aligned(dst, 16))
    return fail(NSR_ERR_BAD_ARG, "calib_copy_rows: rows of a positive multiple of 16 bytes, 16-byte aligned");
  if (n_rows == 0) return NSR_OK;
  DeviceModule* dm = nullptr;
  nsr_status st = current_module(&dm);
  if (st != NSR_OK) return st;
  nsr_calib_args a;
  a.src = (const float*)src;
  a.dst = (float*)dst;
  a.n4 = row_bytes / 16;
  void* params[] = {&a, &n_rows};
  return launch(K_nsrk_calib_copy_rows, (unsigned)std::min<int64_t>(n_rows, dm->n_cu), 1, 512, 0, stream, params);
}

nsr_status nsr_calib_adain_timeline(const float* x, const float* gamma, const float* beta, const float* alpha,
                                    float* out, int64_t B, int64_t C, int64_t T, uint64_t* stamps,
                                    int64_t stamps_words, nsr_stream_t stream) {
  if (!x || !gamma || !beta || !alpha || !out || !stamps)
    return fail(NSR_ERR_BAD_ARG, "calib_adain_timeline: null pointer");
  // the c4b row kernel's bucket only: 57 slots of 512 lanes x 16 bytes (19 in LDS, 38 in VGPRs)
  if (B <= 0 || C <= 0 || B * C > 0x7fffffffLL || T % 4 != 0 || T / 4 <= 512 * 56 || T / 4 > 512 * 57 ||
      !aligned(x, 16) || !aligned(out, 16))
    return fail(NSR_ERR_BAD_ARG,
                "calib_adain_timeline: rows of 114692..116736 floats (T %% 4 == 0), 16-byte aligned, B, C > 0");
  DeviceModule* dm = nullptr;
  nsr_status st = current_module(&dm);
  if (st != NSR_OK) return st;
  const unsigned lds = 19u * 512u * 16u;
  if (lds + 1024 > (unsigned)dm->max_lds) return fail(NSR_ERR_UNSUPPORTED, "calib_adain_timeline: LDS too small");
  const KId kid = K_nsrk_adain_row_tl_b512_v38_l19;
  const int64_t n_rows = B * C;
  const unsigned grid = (unsigned)std::min<int64_t>(n_rows, (int64_t)occupancy(dm, kid, 512, lds) * dm->n_cu);
  if (stamps_words < (int64_t)grid * NSR_ADAIN_TL_WORDS)
    return fail(NSR_ERR_BAD_ARG, "calib_adain_timeline: stamps need %lld words (%u workgroups x %d)",
                (long long)grid * NSR_ADAIN_TL_WORDS, grid, NSR_ADAIN_TL_WORDS);
  nsr_adain_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x;
  a.gamma = gamma;
  a.beta = beta;
  a.alpha = alpha;
  a.out = out;
  a.n_rows = n_rows;
  a.T = T;
  a.gamma_bstride = C;
  a.beta_bstride = C;
  a.C = (int32_t)C;
  a.lds_chunks = 19;
  a.eps = 1e-5f;
  a.inv_t = 1.0f / (float)T;
  a.stamps = stamps;
  int pdt = 0;
  void* params[] = {&a, &pdt};
  return launch(kid, grid, 1, 512, lds, stream, params);
}

}  // extern "C"
