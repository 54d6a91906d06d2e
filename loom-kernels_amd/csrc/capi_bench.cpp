// Eager µs per paged-decode command through the C ABI alone (no Python on the
// per-call path): the caller a Rust or C++ engine would be.  Built next to the
// library by build_lib.sh (loom-kernels_amd/lib/capi_bench) and run by bench.py
// as a child process.
//
//   capi_bench B POOL HQ HKV "indptr,..." "indices,..." "last,..." [SAMPLES]
//   capi_bench --empty-kernel [SAMPLES]
//   capi_bench --graph-floor [SAMPLES]
//
// The second form times an empty kernel launched with hipLaunchKernelGGL the
// same way: the platform's floor for one launch per command.
// Synthetic BF16 inputs (the values do not change the work); the page table is
// the caller's.  Protocol of the reference's eager_stream_batch_cuda_event
// (crates/loom-infer-validation/src/benchmarks/matched.rs:141-173): a hipEvent
// pair around 100 back-to-back enqueues on one stream, divided by 100; the
// median of SAMPLES such batches (default 30) after a warm-up batch.  Also
// reports the host time per enqueue call.  Prints one JSON object.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "loom_infer_hip.h"

namespace {

std::vector<int32_t> parse_list(const char *s) {
  std::vector<int32_t> v;
  std::string cur;
  for (const char *p = s;; ++p) {
    if (*p == ',' || *p == '\0') {
      if (!cur.empty()) v.push_back((int32_t)std::strtol(cur.c_str(), nullptr, 10));
      cur.clear();
      if (*p == '\0') break;
    } else {
      cur.push_back(*p);
    }
  }
  return v;
}

[[noreturn]] void die(const char *what, const loom_error_t &e) {
  std::fprintf(stderr, "capi_bench: %s failed: %s\n", what, e.message);
  std::exit(1);
}

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "capi_bench: %s: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

template <class T>
T *device_copy(const std::vector<T> &h) {
  T *d = nullptr;
  hip_check(hipMalloc(&d, std::max<size_t>(1, h.size()) * sizeof(T)), "hipMalloc");
  if (!h.empty()) hip_check(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "copy");
  return d;
}

__global__ void empty_kernel(int *p) {
  if (p) p[0] = 0;
}

int empty_kernel_floor(int samples) {
  constexpr int kBatch = 100;
  hipStream_t stream;
  hip_check(hipStreamCreate(&stream), "stream");
  hipEvent_t ev0, ev1;
  hip_check(hipEventCreate(&ev0), "event");
  hip_check(hipEventCreate(&ev1), "event");
  std::vector<double> us, host_us;
  for (int s = 0; s <= samples; ++s) {
    hip_check(hipEventRecord(ev0, stream), "record");
    const auto h0 = std::chrono::steady_clock::now();
    for (int i = 0; i < kBatch; ++i)
      hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, stream, nullptr);
    const auto h1 = std::chrono::steady_clock::now();
    hip_check(hipEventRecord(ev1, stream), "record");
    hip_check(hipEventSynchronize(ev1), "sync");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, ev0, ev1), "elapsed");
    if (s > 0) {
      us.push_back(ms * 1000.0 / kBatch);
      host_us.push_back(std::chrono::duration<double, std::micro>(h1 - h0).count() / kBatch);
    }
  }
  std::sort(us.begin(), us.end());
  std::sort(host_us.begin(), host_us.end());
  std::printf("{\"eager_us\": %.3f, \"host_enqueue_us\": %.3f, \"samples\": %d}\n",
              us[us.size() / 2], host_us[host_us.size() / 2], (int)us.size());
  return 0;
}

// Where one graph replay's time goes, with no profiler attached: an empty
// kernel launched eagerly and as a captured one-node hipGraph, each followed
// by an event and a wait for it.  Per form (medians over SAMPLES): the
// GPU-side time between an event recorded before the launch call and one
// after it, the host time inside the launch call, and the host time from
// before the launch call until the wait returns.
int graph_floor(int samples) {
  hipStream_t stream;
  hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "stream");
  hipEvent_t ev0, ev1;
  hip_check(hipEventCreate(&ev0), "event");
  hip_check(hipEventCreate(&ev1), "event");
  hipGraph_t graph = nullptr;
  hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "capture");
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, stream, nullptr);
  hip_check(hipStreamEndCapture(stream, &graph), "capture end");
  hipGraphExec_t exec = nullptr, exec_up = nullptr;
  hip_check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate");
  hip_check(hipGraphInstantiate(&exec_up, graph, nullptr, nullptr, 0), "instantiate");
  hip_check(hipGraphUpload(exec_up, stream), "upload");
  hip_check(hipStreamSynchronize(stream), "sync");
  auto measure = [&](auto launch) {
    std::vector<double> gpu, call, wall;
    for (int s = 0; s < samples + 5; ++s) {
      hip_check(hipEventRecord(ev0, stream), "record");
      const auto h0 = std::chrono::steady_clock::now();
      launch();
      const auto h1 = std::chrono::steady_clock::now();
      hip_check(hipEventRecord(ev1, stream), "record");
      hip_check(hipEventSynchronize(ev1), "sync");
      const auto h2 = std::chrono::steady_clock::now();
      float ms = 0.f;
      hip_check(hipEventElapsedTime(&ms, ev0, ev1), "elapsed");
      if (s >= 5) {
        gpu.push_back(ms * 1000.0);
        call.push_back(std::chrono::duration<double, std::micro>(h1 - h0).count());
        wall.push_back(std::chrono::duration<double, std::micro>(h2 - h0).count());
      }
    }
    for (auto *v : {&gpu, &call, &wall}) std::sort(v->begin(), v->end());
    char buf[256];
    std::snprintf(buf, sizeof buf, "{\"event_us\": %.3f, \"launch_call_us\": %.3f, \"wall_us\": %.3f}",
                  gpu[gpu.size() / 2], call[call.size() / 2], wall[wall.size() / 2]);
    return std::string(buf);
  };
  const std::string eager = measure([&] {
    hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, stream, nullptr);
  });
  const std::string replay = measure([&] { hip_check(hipGraphLaunch(exec, stream), "launch"); });
  const std::string uploaded = measure([&] { hip_check(hipGraphLaunch(exec_up, stream), "launch"); });
  const char *pc = std::getenv("DEBUG_CLR_GRAPH_PACKET_CAPTURE");
  std::printf("{\"eager_one_kernel\": %s, \"graph_one_node\": %s, \"graph_one_node_uploaded\": %s, "
              "\"DEBUG_CLR_GRAPH_PACKET_CAPTURE\": \"%s\", \"samples\": %d}\n",
              eager.c_str(), replay.c_str(), uploaded.c_str(), pc ? pc : "unset", samples);
  (void)hipGraphExecDestroy(exec);
  (void)hipGraphExecDestroy(exec_up);
  (void)hipGraphDestroy(graph);
  return 0;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc >= 2 && std::string(argv[1]) == "--empty-kernel")
    return empty_kernel_floor(argc > 2 ? std::atoi(argv[2]) : 30);
  if (argc >= 2 && std::string(argv[1]) == "--graph-floor")
    return graph_floor(argc > 2 ? std::atoi(argv[2]) : 200);
  if (argc < 8) {
    std::fprintf(stderr, "usage: capi_bench B POOL HQ HKV indptr indices last [samples]\n");
    return 2;
  }
  const uint64_t B = std::strtoull(argv[1], nullptr, 10), pool = std::strtoull(argv[2], nullptr, 10);
  const uint64_t hq = std::strtoull(argv[3], nullptr, 10), hkv = std::strtoull(argv[4], nullptr, 10);
  const std::vector<int32_t> indptr = parse_list(argv[5]), indices = parse_list(argv[6]),
                             last = parse_list(argv[7]);
  const int samples = argc > 8 ? std::atoi(argv[8]) : 30;
  constexpr int kBatch = 100;

  loom_paged_decode_spec_t spec{};
  {
    loom_error_t e{};
    if (loom_paged_decode_spec_new(B, pool, hq, hkv, 128, 16, &spec, &e)) die("spec", e);
  }
  loom_decode_provider_t *prov = nullptr;
  loom_paged_decode_plan_t *plan = nullptr;
  {
    loom_error_t e{};
    if (loom_decode_provider_load(0, &prov, &e)) die("provider", e);
    loom_paged_decode_plan_options_t opt{};
    opt.max_total_pages = indices.size();
    if (loom_decode_provider_plan_bf16_paged_batch(prov, &spec, &opt, &plan, &e)) die("plan", e);
  }
  loom_paged_decode_plan_info_t info{};
  loom_paged_decode_plan_get_info(plan, &info);

  // synthetic bf16 inputs (small LCG values)
  auto bf16_vec = [](size_t n, uint32_t seed) {
    std::vector<uint16_t> v(n);
    for (size_t i = 0; i < n; ++i) {
      seed = seed * 1664525u + 1013904223u;
      v[i] = (uint16_t)(0x3c00 + ((seed >> 20) & 0x1ff));  // values in [2^-7, 2^-6)
    }
    return v;
  };
  const size_t qn = B * hq * 128, kvn = pool * 16 * hkv * 128;
  uint16_t *q = device_copy(bf16_vec(qn, 1)), *k = device_copy(bf16_vec(kvn, 2)),
           *v = device_copy(bf16_vec(kvn, 3));
  int32_t *d_ip = device_copy(indptr), *d_ix = device_copy(indices), *d_ln = device_copy(last);
  uint16_t *out = nullptr;
  float *lse = nullptr;
  hip_check(hipMalloc(&out, qn * 2), "hipMalloc");
  hip_check(hipMalloc(&lse, B * hq * 4), "hipMalloc");

  hipStream_t stream;
  hip_check(hipStreamCreate(&stream), "stream");
  loom_command_queue_t *queue = nullptr;
  loom_bindings_t *b = nullptr;
  loom_bf16_paged_batch_decode_args_t args{};
  {
    loom_error_t e{};
    if (loom_command_queue_new(stream, kBatch + 1, &queue, &e)) die("queue", e);
    if (loom_command_queue_reserve_workspace(queue, info.workspace_bytes, 0, &e)) die("reserve", e);
    if (loom_command_queue_bindings(queue, 8, &b, &e)) die("bindings", e);
    if (loom_bindings_bind_read(b, q, qn, LOOM_DTYPE_BF16, &args.query, &e) ||
        loom_bindings_bind_read(b, k, kvn, LOOM_DTYPE_BF16, &args.key_pages, &e) ||
        loom_bindings_bind_read(b, v, kvn, LOOM_DTYPE_BF16, &args.value_pages, &e) ||
        loom_bindings_bind_read(b, d_ip, indptr.size(), LOOM_DTYPE_I32, &args.page_indptr, &e) ||
        loom_bindings_bind_read(b, d_ix, indices.size(), LOOM_DTYPE_I32, &args.page_indices, &e) ||
        loom_bindings_bind_read(b, d_ln, last.size(), LOOM_DTYPE_I32, &args.last_page_len, &e) ||
        loom_bindings_bind_read_write(b, out, qn, LOOM_DTYPE_BF16, &args.output, &e) ||
        loom_bindings_bind_read_write(b, lse, B * hq, LOOM_DTYPE_F32, &args.lse, &e))
      die("bind", e);
  }
  hipEvent_t ev0, ev1;
  hip_check(hipEventCreate(&ev0), "event");
  hip_check(hipEventCreate(&ev1), "event");
  std::vector<double> us, host_us;
  for (int s = 0; s <= samples; ++s) {
    loom_error_t e{};
    loom_command_scope_t *scope = nullptr;
    if (loom_command_queue_begin(queue, b, &scope, &e)) die("begin", e);
    hip_check(hipEventRecord(ev0, stream), "record");
    const auto h0 = std::chrono::steady_clock::now();
    for (int i = 0; i < kBatch; ++i)
      if (loom_paged_decode_enqueue_bf16(plan, scope, &args, &e)) die("enqueue", e);
    const auto h1 = std::chrono::steady_clock::now();
    hip_check(hipEventRecord(ev1, stream), "record");
    loom_command_completion_t *c = nullptr;
    if (loom_command_scope_finish(scope, &c, &e)) die("finish", e);
    if (loom_command_completion_wait(c, &b, &e)) die("wait", e);
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, ev0, ev1), "elapsed");
    if (s > 0) {  // the first batch warms up
      us.push_back(ms * 1000.0 / kBatch);
      host_us.push_back(std::chrono::duration<double, std::micro>(h1 - h0).count() / kBatch);
    }
  }
  std::sort(us.begin(), us.end());
  std::sort(host_us.begin(), host_us.end());
  std::printf("{\"eager_us\": %.3f, \"p10_us\": %.3f, \"p90_us\": %.3f, \"host_enqueue_us\": %.3f, "
              "\"algorithm\": %d, \"grid_blocks\": %u, \"samples\": %d}\n",
              us[us.size() / 2], us[us.size() / 10], us[us.size() * 9 / 10],
              host_us[host_us.size() / 2], info.algorithm, info.grid_blocks, (int)us.size());
  loom_bindings_free(b);
  loom_command_queue_free(queue);
  loom_paged_decode_plan_free(plan);
  loom_decode_provider_free(prov);
  return 0;
}
