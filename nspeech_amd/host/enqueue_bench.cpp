// Host cost of one call of a C-ABI entry point: the time the calling thread
// spends in the call (argument checks, kernel selection, hipModuleLaunchKernel),
// measured in C++ so that no binding overhead is counted. The decoder-step
// entry points (called per layer per token by the reference's decoder,
// src/moonshine/gpu_decoder.rs:483, gpu_decoder_metal.rs:144-156) at the
// Moonshine decoder shapes, plus an empty kernel through this library and
// the same empty kernel through a bare hipModuleLaunchKernel as the floor, and
// the decoder-step calls of 24 layers captured into one HIP graph: the host
// cost of a replay, per captured call.
//
// Usage: nsr_enqueue_bench <code object dir> [--no-graph]   (prints one JSON object)
// --no-graph leaves out the graph replay: under rocprofv3's kernel trace,
// hipGraphLaunch ended in a segmentation fault inside the tracer on this image.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>

#include "nspeech_rocm.h"

#define CK(x)                                                                                  \
  do {                                                                                         \
    hipError_t e_ = (x);                                                                       \
    if (e_ != hipSuccess) {                                                                    \
      std::fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_));           \
      std::exit(1);                                                                            \
    }                                                                                          \
  } while (0)
#define NK(x)                                                                                  \
  do {                                                                                         \
    nsr_status s_ = (x);                                                                       \
    if (s_ != NSR_OK) {                                                                        \
      std::fprintf(stderr, "%s:%d nsr status %d: %s\n", __FILE__, __LINE__, (int)s_, nsr_last_error()); \
      std::exit(1);                                                                            \
    }                                                                                          \
  } while (0)

static void* dalloc(size_t bytes) {
  void* p = nullptr;
  CK(hipMalloc(&p, bytes));
  CK(hipMemset(p, 0, bytes));
  return p;
}

// Median over batches of the mean host time per call (us). Each batch is
// short enough that the GPU queue never fills, and the stream is drained
// between batches, so the time is the caller's, not a wait for queue space.
static double host_us(hipStream_t s, const std::function<void()>& call, int kBatch = 64) {
  const int kBatches = 31;
  for (int i = 0; i < 2 * kBatch; ++i) call();
  CK(hipStreamSynchronize(s));
  std::vector<double> per;
  for (int b = 0; b < kBatches; ++b) {
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < kBatch; ++i) call();
    const auto t1 = std::chrono::steady_clock::now();
    per.push_back(std::chrono::duration<double, std::micro>(t1 - t0).count() / kBatch);
    CK(hipStreamSynchronize(s));
  }
  std::sort(per.begin(), per.end());
  return per[per.size() / 2];
}

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s <code object dir> [--no-graph]\n", argv[0]);
    return 2;
  }
  const bool graph_replay = !(argc > 2 && std::string(argv[2]) == "--no-graph");
  CK(hipSetDevice(0));
  NK(nsr_init(nullptr));
  hipStream_t s;
  CK(hipStreamCreate(&s));

  // the empty kernel through a bare hipModuleLaunchKernel: the floor of any launch
  hipModule_t mod;
  hipFunction_t fempty;
  CK(hipModuleLoad(&mod, (std::string(argv[1]) + "/nsr_calib_gfx950.hsaco").c_str()));
  CK(hipModuleGetFunction(&fempty, mod, "nsrk_calib_empty"));
  struct {
    const void* a;
    void* b;
    int64_t n;
  } eargs = {nullptr, nullptr, 0};
  void* eparams[] = {&eargs};
  const double raw = host_us(s, [&] { CK(hipModuleLaunchKernel(fempty, 1, 1, 1, 256, 1, 1, 0, s, eparams, nullptr)); });
  const double empty = host_us(s, [&] { NK(nsr_calib_empty(s)); });

  // Moonshine decoder step shapes (kernel_configs.py:102-104): 10 heads x 64, rot 32, cache 448
  const int64_t H = 10, Dh = 64, L = 448, rot = 32, pos = 300;
  void* q = dalloc(H * Dh * 2);
  void* k = dalloc(H * Dh * 2);
  void* v = dalloc(H * Dh * 2);
  void* ck = dalloc(H * L * Dh * 2);
  void* cv = dalloc(H * L * Dh * 2);
  void* tab = dalloc(L * rot * 4);
  void* o = dalloc(H * Dh * 2);
  const double dec = host_us(s, [&] {
    NK(nsr_rope_qk_cache_append(q, k, v, NSR_F16, (const float*)tab, L, ck, cv, H, H, Dh, (int)rot, pos, L, s));
  });
  const double attn = host_us(s, [&] {
    NK(nsr_attention_decode_f16(q, ck, cv, o, L, Dh, H, H, 0.125f, L * Dh, Dh, s));
  });
  // decoder MLP fc1 + bias + GLU over t4 tiles: x f16 [640] @ W [640, 2 x 2560]
  const int64_t K = 640, N = 2560;
  void* x = dalloc(K * 2);
  void* tq = dalloc(K * 2 * N);
  void* ts = dalloc(K / 32 * 2 * N * 2);
  void* bias = dalloc(2 * N * 4);
  void* out = dalloc(N * 2);
  const double q8fc1 = host_us(s, [&] {
    NK(nsr_gemv_q8_t4_bias_glu(x, NSR_F16, (const uint32_t*)tq, (const uint16_t*)ts, (const float*)bias, out,
                               NSR_F16, K, N, s));
  });
  CK(hipStreamSynchronize(s));

  // The same three calls per layer for 24 decoder layers, captured once into a HIP graph (the entry points
  // only launch kernels: no allocation, synchronisation or memset) and replayed: the host cost of a
  // replay, per captured call. Batches of 4 replays keep the queue from filling.
  const int kLayers = 24;
  std::printf(
      "{\"unit\": \"us per call, host\", \"hipModuleLaunchKernel_empty\": %.3f, \"nsr_calib_empty\": %.3f, "
      "\"dec\": %.3f, \"attn\": %.3f, \"q8fc1\": %.3f",
      raw, empty, dec, attn, q8fc1);
  if (graph_replay) {
    hipGraph_t graph;
    hipGraphExec_t exec;
    CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
    for (int l = 0; l < kLayers; ++l) {
      NK(nsr_rope_qk_cache_append(q, k, v, NSR_F16, (const float*)tab, L, ck, cv, H, H, Dh, (int)rot, pos, L, s));
      NK(nsr_attention_decode_f16(q, ck, cv, o, L, Dh, H, H, 0.125f, L * Dh, Dh, s));
      NK(nsr_gemv_q8_t4_bias_glu(x, NSR_F16, (const uint32_t*)tq, (const uint16_t*)ts, (const float*)bias, out,
                                 NSR_F16, K, N, s));
    }
    CK(hipStreamEndCapture(s, &graph));
    CK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    const double replay = host_us(s, [&] { CK(hipGraphLaunch(exec, s)); }, 4);
    CK(hipStreamSynchronize(s));
    CK(hipGraphExecDestroy(exec));
    CK(hipGraphDestroy(graph));
    std::printf(", \"graph_replay_per_call\": %.3f, \"graph_replay\": %.3f, \"graph_calls\": %d",
                replay / (3.0 * kLayers), replay, 3 * kLayers);
  }
  std::printf("}\n");
  return 0;
}
