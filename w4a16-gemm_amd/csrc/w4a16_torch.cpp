// PyTorch-ROCm binding: module `w4a16_opt`, function `w4a16_gemm(Wp, x, scales, variant=-1)`.
//
// Drop-in for the reference's pybind11 entry point (src/vectorized/extension.cpp:5-9) and the
// tensor-level half of w4a16_gemm_cuda (src/vectorized/kernel.cu:218-267).  All numeric
// validation, routing, tile selection and the kernel launches go through the C ABI of
// libw4a16_hip.so (include/w4a16.h); this file only owns tensors, the device guard, the current
// stream, the output allocation and the split-K scratch.
//
// Compiled by the host compiler (no hipify, no device code).
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <chrono>
#include <initializer_list>
#include <vector>
#include <map>
#include <mutex>

#include <string>

#include "w4a16.h"
#include "w4a16_internal.h"

namespace {

// Split-K counters (decode split-K and the long-K prefill token-group configs, which run one
// K segment per workgroup).  Launches that share a counter buffer must not overlap in time
// (w4a16.h), and work on different streams may overlap, so:
//  * eager calls keep one buffer per (device, stream): zeroed when created, left zero by every
//    launch;
//  * a call made under HIP graph capture gets a slice of its own from a per-device pool that the
//    first eager call on the device zeroed; a slice is never handed out again, so graph nodes and
//    eager work never share counters, and every replay leaves its slice zero for the next one.
//    A graph must not be replayed concurrently with itself (its nodes own their slices).
//  * if the pool is missing (no eager call before the capture) or used up, the captured call
//    allocates its counters from the capture's memory pool and zeroes them with a fill kernel
//    that the graph records (correct, one extra graph node per such call).
// The returned tensor must stay alive until the launch is enqueued.
constexpr int64_t kCapturePoolSlots = 1 << 20;

struct CapturePool {
    at::Tensor buf;
    int64_t next = 0;
};

std::mutex g_mu;
std::map<std::pair<int, hipStream_t>, at::Tensor> g_counters;
std::map<int, CapturePool> g_capture_pool;
// Set once a device's pool exists (cleared by the test hook that drops it): lets every later
// call skip the capture-status query that guards the pool's creation (~0.16 us per call).
constexpr int kMaxPoolDevices = 64;
std::atomic<bool> g_pool_ready[kMaxPoolDevices];

bool pool_ready(int dev) {
    return dev >= 0 && dev < kMaxPoolDevices && g_pool_ready[dev].load(std::memory_order_acquire);
}

bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    TORCH_CHECK(hipStreamIsCapturing(stream, &st) == hipSuccess, "hipStreamIsCapturing failed");
    return st != hipStreamCaptureStatusNone;
}

// Called on every eager call: creates the device's capture pool once, outside any capture.
void ensure_capture_pool(const at::Tensor& like) {
    const int dev = (int)like.device().index();
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_capture_pool.count(dev)) {
        at::Tensor buf = torch::zeros({kCapturePoolSlots}, like.options().dtype(torch::kInt32));
        // The zero fill runs on the current stream, and captured launches may later run on another
        // one: wait for the fill alone, once per device, through an event (a stream or device
        // synchronisation would invalidate a capture running on another stream in global mode).
        hipEvent_t ev = nullptr;
        TORCH_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess, "w4a16_gemm: hipEventCreate failed");
        const bool ok = hipEventRecord(ev, c10::hip::getCurrentHIPStream(dev).stream()) == hipSuccess &&
                        hipEventSynchronize(ev) == hipSuccess;
        (void)hipEventDestroy(ev);
        TORCH_CHECK(ok, "w4a16_gemm: waiting for the capture pool's zero fill failed");
        g_capture_pool[dev].buf = buf;
    }
    if (dev >= 0 && dev < kMaxPoolDevices) g_pool_ready[dev].store(true, std::memory_order_release);
}

// Test hook: forget the capture pool of a device, so that the next call under capture takes the
// no-pool path (counters zeroed by a fill kernel recorded in the graph).  The dropped buffer is
// kept alive: graphs captured before the drop hold pointers into it and may still be replayed.
std::vector<at::Tensor> g_dropped_pools;

void drop_capture_pool(int64_t device) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_capture_pool.find((int)device);
    if (it == g_capture_pool.end()) return;
    if (device >= 0 && device < kMaxPoolDevices) g_pool_ready[device].store(false, std::memory_order_release);
    g_dropped_pools.push_back(it->second.buf);
    g_capture_pool.erase(it);
}

at::Tensor split_counters(const at::Tensor& like, hipStream_t stream, int32_t slots) {
    const auto opts = like.options().dtype(torch::kInt32);
    const int dev = (int)like.device().index();
    std::lock_guard<std::mutex> lk(g_mu);
    if (capturing(stream)) {
        auto pit = g_capture_pool.find(dev);
        if (pit != g_capture_pool.end() && pit->second.next + slots <= kCapturePoolSlots) {
            at::Tensor slice = pit->second.buf.narrow(0, pit->second.next, slots);
            pit->second.next += (slots + 63) / 64 * 64;          // 256-byte aligned slices
            return slice;
        }
        return torch::zeros({(int64_t)slots}, opts);
    }
    const std::pair<int, hipStream_t> key{dev, stream};
    auto it = g_counters.find(key);
    if (it == g_counters.end())
        it = g_counters.emplace(key, torch::zeros({(int64_t)w4a16_max_counter_slots()}, opts)).first;
    return it->second;
}

w4a16_device_limits limits_for(int dev) {
    w4a16_device_limits lim;
    const int rc = w4a16_query_device(dev, &lim);
    TORCH_CHECK(rc == W4A16_OK, "w4a16_gemm: device query failed: ", w4a16_last_error());
    return lim;
}

}  // namespace

torch::Tensor w4a16_gemm(torch::Tensor Wp, torch::Tensor x, torch::Tensor scales, int64_t variant) {
    // kernel.cu:219-223 (same order, same messages; ROCm tensors report is_cuda()).
    TORCH_CHECK(Wp.is_cuda() && x.is_cuda() && scales.is_cuda(), "all tensors must be CUDA");
    TORCH_CHECK(Wp.is_contiguous() && x.is_contiguous() && scales.is_contiguous(), "contiguous only");
    TORCH_CHECK(Wp.dtype() == torch::kInt32, "Wp must be int32");
    TORCH_CHECK(x.dtype() == torch::kHalf && scales.dtype() == torch::kHalf, "x, scales must be fp16");
    TORCH_CHECK(x.dim() == 2 && scales.dim() == 2, "x must be [M, K], scales must be [K/G, N]");

    w4a16_problem prob;
    prob.M = x.size(0);
    prob.K = x.size(1);
    prob.N = scales.size(1);
    prob.groups = scales.size(0);
    prob.wp_words = Wp.numel();
    prob.Wp = Wp.data_ptr();
    prob.x = x.data_ptr();
    prob.scales = scales.data_ptr();

    const c10::DeviceGuard guard(x.device());
    const int dev = x.device().index();
    const w4a16_device_limits lim = limits_for(dev);
    w4a16_plan plan;
    char err[512];
    const int rc = w4a16_plan_create(&prob, (int)std::max<int64_t>(std::min<int64_t>(variant, 1 << 20), -(1 << 20)),
                                     &lim, &plan, err, sizeof(err));
    TORCH_CHECK(rc == W4A16_OK, err);
    TORCH_CHECK(Wp.device() == x.device() && scales.device() == x.device(),
                "Wp, x and scales must be on the same device");

    hipStream_t stream = c10::hip::getCurrentHIPStream(dev).stream();
    torch::Tensor y = torch::empty({prob.M, prob.N}, x.options());
    if (y.numel() == 0) return y;
    if (!pool_ready(dev) && !capturing(stream)) ensure_capture_pool(x);

    torch::Tensor ws;
    void* ws_ptr = nullptr;
    if (plan.workspace_bytes) {
        ws = torch::empty({(int64_t)plan.workspace_bytes}, x.options().dtype(torch::kUInt8));
        ws_ptr = ws.data_ptr();
    }
    torch::Tensor cnt_t;
    int32_t* cnt = nullptr;
    if (plan.counter_slots) {
        cnt_t = split_counters(x, stream, plan.counter_slots);
        cnt = cnt_t.data_ptr<int32_t>();
    }

    const int lrc = w4a16_launch(&plan, static_cast<const int32_t*>(prob.Wp),
                                 static_cast<const uint16_t*>(prob.x), static_cast<const uint16_t*>(prob.scales),
                                 reinterpret_cast<uint16_t*>(y.data_ptr()), ws_ptr, cnt, stream);
    TORCH_CHECK(lrc == W4A16_OK, "w4a16_gemm: launch failed (code ", lrc, "): ", w4a16_last_error());
    return y;
}

// Measurement hook (bench.py's eager leg): host microseconds per step of the eager call path,
// each step timed over `reps` repetitions with the steady clock; the launches are real (the
// caller synchronises afterwards).
py::dict w4a16_host_breakdown(torch::Tensor Wp, torch::Tensor x, torch::Tensor scales, int64_t reps) {
    using clk = std::chrono::steady_clock;
    auto us = [&](clk::time_point a, clk::time_point b) {
        return std::chrono::duration<double, std::micro>(b - a).count() / (double)reps;
    };
    w4a16_problem prob;
    prob.M = x.size(0); prob.K = x.size(1); prob.N = scales.size(1); prob.groups = scales.size(0);
    prob.wp_words = Wp.numel(); prob.Wp = Wp.data_ptr(); prob.x = x.data_ptr(); prob.scales = scales.data_ptr();
    const int dev = x.device().index();
    py::dict d;
    auto t0 = clk::now();
    for (int64_t i = 0; i < reps; ++i) {
        TORCH_CHECK(Wp.is_cuda() && x.is_cuda() && scales.is_cuda(), "all tensors must be CUDA");
        TORCH_CHECK(Wp.is_contiguous() && x.is_contiguous() && scales.is_contiguous(), "contiguous only");
        const c10::DeviceGuard guard(x.device());
    }
    auto t1 = clk::now();
    w4a16_device_limits lim{};
    for (int64_t i = 0; i < reps; ++i) lim = limits_for(dev);
    auto t2 = clk::now();
    w4a16_plan plan;
    char err[512];
    for (int64_t i = 0; i < reps; ++i) TORCH_CHECK(w4a16_plan_create(&prob, -1, &lim, &plan, err, sizeof(err)) == W4A16_OK, err);
    auto t3 = clk::now();
    hipStream_t stream = nullptr;
    for (int64_t i = 0; i < reps; ++i) stream = c10::hip::getCurrentHIPStream(dev).stream();
    auto t4 = clk::now();
    for (int64_t i = 0; i < reps; ++i) {                      // y from the caching allocator, freed again
        torch::Tensor y = torch::empty({prob.M, prob.N}, x.options());
        (void)y;
    }
    auto t5 = clk::now();
    std::vector<torch::Tensor> ys;                            // outputs of the launch step (untimed)
    ys.reserve(reps);
    bool cap = false;                                         // the op's guard of the pool's creation
    for (int64_t i = 0; i < reps; ++i) cap = cap || (!pool_ready(dev) && capturing(stream));
    auto t6 = clk::now();
    for (int64_t i = 0; i < reps; ++i) ys.push_back(torch::empty({prob.M, prob.N}, x.options()));
    auto t7 = clk::now();
    TORCH_CHECK(plan.workspace_bytes == 0 && plan.counter_slots == 0, "host breakdown: unsplit plans only");
    for (int64_t i = 0; i < reps; ++i)
        TORCH_CHECK(w4a16_launch(&plan, static_cast<const int32_t*>(prob.Wp), static_cast<const uint16_t*>(prob.x),
                                 static_cast<const uint16_t*>(prob.scales), reinterpret_cast<uint16_t*>(ys[i].data_ptr()),
                                 nullptr, nullptr, stream) == W4A16_OK, "launch failed");
    auto t8 = clk::now();
    d["checks_and_device_guard"] = us(t0, t1);
    d["device_limits"] = us(t1, t2);
    d["plan_create"] = us(t2, t3);
    d["current_stream"] = us(t3, t4);
    d["allocate_y"] = us(t4, t5);
    d["capture_check"] = us(t5, t6);
    d["launch"] = us(t7, t8);
    return d;
}

// Device quantise + pack: the GPU replacement of the reference's quantize_w4 followed by
// pack_int4 (tests/quant.py:62-74, 34-48).  Returns (Wp int32 [N*K/8], scales fp16 [K/G, N]).
std::tuple<torch::Tensor, torch::Tensor> w4a16_quantize_pack_t(torch::Tensor W, int64_t group_size) {
    TORCH_CHECK(W.is_cuda(), "W must be CUDA");
    TORCH_CHECK(W.is_contiguous(), "contiguous only");
    TORCH_CHECK(W.dtype() == torch::kHalf || W.dtype() == torch::kFloat, "W must be fp16 or fp32");
    TORCH_CHECK(W.dim() == 2, "W must be [N, K]");
    const int64_t N = W.size(0), K = W.size(1);
    TORCH_CHECK(group_size > 0 && K % group_size == 0, "K must be a multiple of the group size");
    const c10::DeviceGuard guard(W.device());
    const int dev = W.device().index();
    torch::Tensor Wp = torch::empty({N * K / 8}, W.options().dtype(torch::kInt32));
    torch::Tensor scales = torch::empty({K / group_size, N}, W.options().dtype(torch::kHalf));
    hipStream_t stream = c10::hip::getCurrentHIPStream(dev).stream();
    const int rc = w4a16_quantize_pack(W.data_ptr(), W.dtype() == torch::kFloat ? 1 : 0, N, K, group_size,
                                       Wp.data_ptr<int32_t>(), reinterpret_cast<uint16_t*>(scales.data_ptr()),
                                       stream);
    TORCH_CHECK(rc == W4A16_OK, "quantize_pack: ", w4a16_last_error());
    return {Wp, scales};
}

// Introspection used by the tests and the benchmark: the plan the op would launch.
py::dict w4a16_plan_info(int64_t M, int64_t N, int64_t K, int64_t G, int64_t variant, int64_t device) {
    w4a16_problem prob;
    prob.M = M; prob.N = N; prob.K = K;
    prob.groups = G > 0 ? K / G : 0;
    prob.wp_words = N * K / 8;
    prob.Wp = prob.x = prob.scales = nullptr;
    const w4a16_device_limits lim = limits_for((int)device);
    w4a16_plan plan;
    char err[512];
    const int rc = w4a16_plan_create(&prob, (int)variant, &lim, &plan, err, sizeof(err));
    TORCH_CHECK(rc == W4A16_OK, err);
    py::dict d;
    d["kernel"] = plan.kernel; d["splits"] = plan.splits; d["slab_chunks"] = plan.slab_chunks;
    d["tile_n"] = plan.tile_n; d["grid"] = plan.grid; d["block"] = plan.block;
    d["counter_slots"] = plan.counter_slots; d["workspace_bytes"] = (uint64_t)plan.workspace_bytes;
    d["decode_variant"] = plan.decode_variant;
    // Names as the compiler demangles them (what rocprofv3 reports), e.g.
    // "w4a16::decode_ring_kernel<2, 4, 2, 1>".
    auto tmpl = [](const char* name, std::initializer_list<int> args, const char* last = nullptr) {
        std::string s = std::string("w4a16::") + name + "<";
        bool first = true;
        for (int a : args) { s += (first ? "" : ", ") + std::to_string(a); first = false; }
        if (last) s += std::string(", ") + last;
        return s + ">";
    };
    if (plan.kernel == W4A16_VARIANT_DECODE) {
        static const char* const kinds[] = {"decode_kernel", "", "decode_stream_kernel", "decode_ring_kernel"};
        const w4a16::DecodeCfg& c = w4a16::kDecodeTable[plan.decode_variant];
        d["kernel_name"] = c.kind == 3 ? tmpl(kinds[3], {c.nbw, c.waves, c.d, w4a16::decode_ring_xr((int)M)})
                                       : tmpl(kinds[c.kind], {c.nbw, c.waves, c.d});
    } else {
        const w4a16::PrefillTile& t = w4a16::kPrefillTable[plan.kernel];
        if (t.kind == 2)
            d["kernel_name"] = tmpl("prefill_stream_kernel", {t.bm / 16, t.depth});
        else if (t.kind == 3)
            d["kernel_name"] = tmpl("prefill_group_kernel", {t.bm / 16, t.depth, t.waves_n, t.bn / (16 * t.waves_n)});
        else {
            // the wide and tiled kernels carry the long-K segment flag as their last template argument
            const bool segs = w4a16::prefill_segments((int)(K / 64)) > 1;
            const char* seg = segs ? "true" : "false";
            if (t.kind == 1) {
                std::string n = tmpl(t.pipe ? "prefill_wide_pipe_kernel" : "prefill_wide_kernel",
                                     {t.bm, t.bn, t.waves_m, t.waves_n, t.wpe}, seg);
                d["kernel_name"] = n.substr(0, n.size() - 1) + ", " +
                                   std::to_string(w4a16::prefill_wide_steps(plan.kernel, segs)) + ">";
            }
            else
                d["kernel_name"] = tmpl("prefill_kernel", {t.bm, t.bn, t.waves_m, t.waves_n}, seg);
        }
    }
    d["cu_count"] = lim.cu_count; d["gcn_arch"] = lim.gcn_arch; d["lds_bytes_per_block"] = lim.lds_bytes_per_block;
    return d;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("w4a16_gemm", &w4a16_gemm,
          "W4A16 group-wise GEMM on MI355X MFMA (decode M<=16 split-K kernel + tiled prefill for any M)",
          py::arg("Wp"), py::arg("x"), py::arg("scales"), py::arg("variant") = -1);
    m.def("plan_info", &w4a16_plan_info, "Plan the op would launch for a shape (debug / bench)",
          py::arg("M"), py::arg("N"), py::arg("K"), py::arg("G"), py::arg("variant") = -1, py::arg("device") = 0);
    m.def("quantize_pack", &w4a16_quantize_pack_t,
          "Group-wise RTN int4 quantisation + packing on the device: W [N, K] -> (Wp, scales)",
          py::arg("W"), py::arg("group_size"));
    m.def("_debug_host_breakdown", &w4a16_host_breakdown,
          "Measurement hook: host microseconds per step of an eager call (unsplit plans)",
          py::arg("Wp"), py::arg("x"), py::arg("scales"), py::arg("reps") = 200);
    m.def("_debug_drop_capture_pool", &drop_capture_pool,
          "Test hook: forget a device's capture pool (the next captured split-K call zeroes its own counters)",
          py::arg("device") = 0);
    m.attr("abi_version") = w4a16_abi_version();
}
