// dllm_hip_sum_squares_noalloc: the exact serial sum of squares of dllm_hip_sum_squares with every scratch buffer
// (the block plan, the block sums and estimates, the block functions and the result) in one file-scope device array,
// for callers that cannot allocate device memory or pass a workspace. Nothing here calls hipMalloc or hipFree.
//
// Each GPU holds its own copy of `scratch` at its own address, found once per device with hipGetSymbolAddress and
// kept in g_scratch[device]; host code only ever passes that address, never the array's name (on the host the name
// is a stand-in, not a device address). Every call on one GPU shares that GPU's array, so the calls on one GPU are
// serialised: each holds that GPU's call lock from its first launch until its stream has finished the result (the
// call waits for its stream before returning anyway), and calls from two host threads or on two streams never
// overlap on the array.
#include <mutex>

#include "common.h"
#include "dllm_hip.h"
#include "kernels.h"
#include "workspace.h"

using namespace dllm_hip;

namespace {

// 65536 blocks of 8192 elements: tensors of up to 2^29 values (2 GiB of float32).
constexpr size_t kMaxBlocks = 65536;
constexpr size_t kBlockElems = static_cast<size_t>(kSumSquaresBlock);
constexpr size_t kMaxValues = kMaxBlocks * kBlockElems;

size_t scratch_layout(size_t blocks) {
    Layout l;
    l.add<int64_t>(2);           // first block, block count
    l.add<int64_t>(2 * blocks);  // block starts and counts
    l.add<char>(exact_sum_squares_workspace(blocks));
    l.add<double>(1);            // the result
    return l.bytes;
}

// 64 bytes per block plus the alignment slack of the layout: 4 MiB + 4 KiB.
constexpr size_t kScratchBytes = kMaxBlocks * 64 + 4096;

}  // namespace

static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_lock;
char* g_scratch[kMaxDevices] = {};
std::mutex g_call[kMaxDevices];  // one call at a time per GPU on its scratch array

// The device address of this GPU's scratch array (looked up on the first call with the device current).
int device_scratch(char** out, int* device_out) {
    int device = 0;
    DLLM_TRY(check_hip(hipGetDevice(&device), "hipGetDevice"));
    DLLM_REQUIRE(device >= 0 && device < kMaxDevices, "sum_squares_noalloc supports devices 0..63");
    std::lock_guard<std::mutex> guard(g_lock);
    if (g_scratch[device] == nullptr) {
        void* p = nullptr;
        DLLM_TRY(check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
        g_scratch[device] = static_cast<char*>(p);
    }
    *out = g_scratch[device];
    *device_out = device;
    return kOk;
}

// The single-tensor plan of exact_sum_squares_plan, written on the device: head = {0, blocks}; block b starts at
// b * 8192 and holds min(8192, n - b * 8192) values (one empty block for n = 0).
__global__ void single_tensor_plan_kernel(int64_t n, int64_t blocks, int64_t* head, int64_t* bstart,
                                          int64_t* bcount) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b == 0) {
        head[0] = 0;
        head[1] = blocks;
    }
    if (b < blocks) {
        const int64_t start = b * static_cast<int64_t>(kBlockElems);
        bstart[b] = start;
        bcount[b] = n > 0 ? (n - start < static_cast<int64_t>(kBlockElems) ? n - start
                                                                            : static_cast<int64_t>(kBlockElems))
                          : 0;
    }
}

}  // namespace

extern "C" int dllm_hip_sum_squares_noalloc(const float* values, size_t n, double* result, void* stream) {
    DLLM_REQUIRE(n <= kMaxValues, "sum_squares_noalloc takes at most 2^29 values (its fixed scratch size); use "
                                  "dllm_hip_sum_squares with a workspace for larger tensors");
    const size_t blocks = n > 0 ? ceil_div(n, kBlockElems) : 1;
    DLLM_REQUIRE(scratch_layout(blocks) <= kScratchBytes, "sum_squares_noalloc scratch layout overflow");
    char* base = nullptr;
    int device = 0;
    DLLM_TRY(device_scratch(&base, &device));
    std::lock_guard<std::mutex> call(g_call[device]);  // until this call's stream has finished with the array
    Carve c(base, kScratchBytes);
    int64_t* d_head = c.take<int64_t>(2);
    int64_t* d_table = c.take<int64_t>(2 * blocks);
    char* ws = c.take<char>(exact_sum_squares_workspace(blocks));
    double* d_result = c.take<double>(1);
    DLLM_REQUIRE(!c.overflow, "sum_squares_noalloc scratch layout overflow");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // Every scratch byte the passes read is written earlier in the same call (plan, block sums, estimates, block
    // functions, result), so the previous call's contents need no clearing.
    const unsigned grid = static_cast<unsigned>(ceil_div(blocks, 256));
    hipLaunchKernelGGL(single_tensor_plan_kernel, dim3(grid), dim3(256), 0, s, static_cast<int64_t>(n),
                       static_cast<int64_t>(blocks), d_head, d_table, d_table + blocks);
    DLLM_TRY(check_launch("sum_squares_noalloc plan"));
    ExactSumPlan plan;
    plan.tensors = 1;
    plan.blocks = static_cast<int64_t>(blocks);
    plan.tfirst = d_head;
    plan.tblocks = d_head + 1;
    plan.bstart = d_table;
    plan.bcount = d_table + blocks;
    DLLM_TRY(launch_exact_sum_squares(values, plan, ws, d_result, s));
    double host = 0.0;
    DLLM_TRY(check_hip(hipMemcpyAsync(&host, d_result, sizeof host, hipMemcpyDeviceToHost, s), "download"));
    DLLM_TRY(check_hip(hipStreamSynchronize(s), "sum_squares_noalloc"));
    if (result) *result = host;
    return kOk;
}
