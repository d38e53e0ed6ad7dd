// C-ABI entry points of libattn_mi355x.so (declared in include/attn_mi355x.h).
// Argument checking and no-op rules mirror the reference launchers; kernels
// are chosen per shape (MFMA/vector paths for the SmolLM3 shapes, generic
// kernels for everything else).  Nothing here allocates device memory, so
// every launch can be captured into a HIP graph.
#include "attn_internal.hpp"
#include "../../include/attn_mi355x.h"

#include <atomic>
#include <cmath>
#include <cstring>
#include <functional>
#include <mutex>
#include <unordered_map>

namespace attn {

namespace {

std::atomic<long> g_options[kOptCount];

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

hipError_t captured_node(hipStream_t stream, hipGraphNode_t* out) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    const hipGraphNode_t* deps = nullptr;
    size_t count = 0;
    hipError_t e = hipStreamGetCaptureInfo_v2(stream, &status, nullptr, nullptr, &deps, &count);
    if (e != hipSuccess) return e;
    // gpu_utils.hpp:45-59: exactly one capture dependency is expected
    if (status != hipStreamCaptureStatusActive || count != 1 || deps == nullptr)
        return hipErrorIllegalState;
    *out = deps[0];
    return hipSuccess;
}

bool fits_u32(size_t v) { return v <= 0xffffffffull; }

// What a merge node's kernel reads from its arguments, last written into each
// (graph exec, merge node) pair by update_merge_attention_decode_node or
// update_rope_and_store_kv_decode_nodes.  The merge kernels read only the
// state count, the whole-context flag (which also sets the grid), the
// rotation switch and buffer pointers that never change
// (the fused RoPE form takes the position from the word the split kernel
// leaves), so a patch that keeps count and switch is skipped -- but only when
// they also equal the node's captured ones: an exec node holds either its
// captured arguments or the last ones patched in, which this table records,
// and a stale entry (a destroyed exec's handle reused) can then only cause a
// redundant patch, never a skipped one.  hipGraphExecKernelNodeSetParams
// costs ~0.6 us of host time per call.
struct MergePatchKey {
    hipGraphExec_t exec;
    hipGraphNode_t node;
    bool operator==(const MergePatchKey& o) const { return exec == o.exec && node == o.node; }
};
struct MergePatchHash {
    size_t operator()(const MergePatchKey& k) const {
        return std::hash<const void*>()(k.exec) * 31u ^ std::hash<const void*>()(k.node);
    }
};
std::mutex g_merge_mu;
std::unordered_map<MergePatchKey, uint64_t, MergePatchHash> g_merge_sig;
constexpr size_t kMergeTableMax = 1u << 16;  // cleared when full (only costs patches)

uint64_t merge_sig(const DecodeArgs& a) {
    return (uint64_t)a.nstate << 2 | (a.whole ? 2u : 0u) | (a.apply ? 1u : 0u);
}

// whether the exec node already runs the merge with `sig`, captured with
// `captured`
bool merge_current(hipGraphExec_t exec, hipGraphNode_t node, uint64_t captured, uint64_t sig) {
    if (sig != captured) return false;
    std::lock_guard<std::mutex> lock(g_merge_mu);
    const auto it = g_merge_sig.find(MergePatchKey{exec, node});
    return it == g_merge_sig.end() || it->second == sig;
}

void merge_patched(hipGraphExec_t exec, hipGraphNode_t node, uint64_t sig) {
    std::lock_guard<std::mutex> lock(g_merge_mu);
    if (g_merge_sig.size() >= kMergeTableMax) g_merge_sig.clear();
    g_merge_sig[MergePatchKey{exec, node}] = sig;
}

// Kernel nodes remembered at capture, so that the graph updaters patch a node
// without reading it back (hipGraphKernelNodeGetParams, ~0.07 us per call;
// the reference updaters read the node back on every call,
// causal_attention.hip.cpp:981,1009, rope.hip.cpp:215).  Every kernel
// launched here while its stream is capturing is recorded with its launch
// configuration and its one struct argument as captured, tagged with a serial
// of the graph being captured.  The first record of a graph retains a user
// object on that graph whose release drops the graph's records, so a node
// handle the runtime hands out again after the graph is destroyed never meets
// a record of the old node.  Nodes without a record (cloned graphs, a failed
// lookup at capture, records switched off with the option
// "graph_node_records" = 1) are read back as before.  The store is allocated
// once and never freed, so a release during process teardown still finds it.
constexpr size_t kNodeArgMax = 512;
constexpr size_t kNodeRecordsMax = 1u << 16;  // cleared when full (only costs read-backs)
struct NodeRecord {
    uint64_t serial;
    int device;  // the capturing stream's device
    const void* func;
    dim3 grid, block;
    unsigned shmem;
    uint32_t arg_bytes;
    alignas(16) unsigned char arg[kNodeArgMax];
};
struct NodeStore {
    std::mutex mu;
    std::unordered_map<hipGraphNode_t, NodeRecord> nodes;
    std::unordered_map<hipGraph_t, uint64_t> graphs;  // graphs holding a user object
    uint64_t next_serial = 1;
};
NodeStore& node_store() {
    static NodeStore* store = new NodeStore;
    return *store;
}
struct GraphTag {
    hipGraph_t graph;
    uint64_t serial;
};

// user-object destructor: runs when the graph and its executable graphs are
// released; it makes no HIP call
void drop_graph_records(void* p) {
    GraphTag* tag = static_cast<GraphTag*>(p);
    NodeStore& s = node_store();
    {
        std::lock_guard<std::mutex> lock(s.mu);
        for (auto it = s.nodes.begin(); it != s.nodes.end();)
            it = it->second.serial == tag->serial ? s.nodes.erase(it) : std::next(it);
        const auto g = s.graphs.find(tag->graph);
        if (g != s.graphs.end() && g->second == tag->serial) s.graphs.erase(g);
    }
    delete tag;
}

// The serial of a graph under capture, retaining the user object the first
// time; 0 when the runtime refuses it (then nothing is recorded).
uint64_t graph_serial(hipGraph_t graph) {
    NodeStore& s = node_store();
    uint64_t serial = 0;
    {
        std::lock_guard<std::mutex> lock(s.mu);
        const auto it = s.graphs.find(graph);
        if (it != s.graphs.end()) return it->second;
        serial = s.next_serial++;
    }
    GraphTag* tag = new GraphTag{graph, serial};
    hipUserObject_t obj = nullptr;
    if (hipUserObjectCreate(&obj, tag, drop_graph_records, 1, hipUserObjectNoDestructorSync) !=
        hipSuccess) {
        delete tag;
        return 0;
    }
    if (hipGraphRetainUserObject(graph, obj, 1, hipGraphUserObjectMove) != hipSuccess) {
        (void)hipUserObjectRelease(obj, 1);  // runs drop_graph_records, which frees tag
        return 0;
    }
    std::lock_guard<std::mutex> lock(s.mu);
    return s.graphs.emplace(graph, serial).first->second;
}

// After a launch on `stream`: if the stream is capturing, record the node the
// launch added.  Args is the kernel's one struct argument.
template <class Args>
void remember_launch(hipStream_t stream) {
    static_assert(sizeof(Args) <= kNodeArgMax, "node argument larger than a record");
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    hipGraph_t graph = nullptr;
    const hipGraphNode_t* deps = nullptr;
    size_t count = 0;
    if (hipStreamGetCaptureInfo_v2(stream, &status, nullptr, &graph, &deps, &count) !=
            hipSuccess ||
        status != hipStreamCaptureStatusActive || count != 1 || !deps || !graph)
        return;
    const hipGraphNode_t node = deps[0];
    hipKernelNodeParams p{};
    if (hipGraphKernelNodeGetParams(node, &p) != hipSuccess || !p.kernelParams || !p.func) return;
    hipDevice_t device = 0;
    if (hipStreamGetDevice(stream, &device) != hipSuccess) return;
    NodeRecord r;
    r.device = (int)device;
    r.func = p.func;
    r.grid = p.gridDim;
    r.block = p.blockDim;
    r.shmem = p.sharedMemBytes;
    r.arg_bytes = (uint32_t)sizeof(Args);
    std::memcpy(r.arg, p.kernelParams[0], sizeof(Args));
    r.serial = graph_serial(graph);
    if (r.serial == 0) return;
    NodeStore& s = node_store();
    std::lock_guard<std::mutex> lock(s.mu);
    if (s.nodes.size() >= kNodeRecordsMax) s.nodes.clear();
    s.nodes[node] = r;
}

// A kernel node as an updater sees it: launch configuration and a pointer to
// its one struct argument (a private copy, or the node's own storage when it
// had to be read back).
struct NodeView {
    hipKernelNodeParams params{};
    const void* arg = nullptr;
    int device = -1;  // recorded nodes: the device they were captured on
    alignas(16) unsigned char copy[kNodeArgMax];
};

hipError_t view_node(hipGraphNode_t node, NodeView& v) {
    if (get_option(kOptGraphNodeRecords) != 1) {
        NodeStore& s = node_store();
        std::lock_guard<std::mutex> lock(s.mu);
        const auto it = s.nodes.find(node);
        if (it != s.nodes.end()) {
            const NodeRecord& r = it->second;
            v.params = hipKernelNodeParams{};
            v.params.func = const_cast<void*>(r.func);
            v.params.gridDim = r.grid;
            v.params.blockDim = r.block;
            v.params.sharedMemBytes = r.shmem;
            std::memcpy(v.copy, r.arg, r.arg_bytes);
            v.arg = v.copy;
            v.device = r.device;
            return hipSuccess;
        }
    }
    v.params = hipKernelNodeParams{};
    const hipError_t e = hipGraphKernelNodeGetParams(node, &v.params);
    if (e != hipSuccess) return e;
    if (!v.params.kernelParams) return hipErrorInvalidValue;
    v.arg = v.params.kernelParams[0];
    return hipSuccess;
}

// The device a node's plan is made for: its capturing stream's when recorded,
// else the current one.
hipError_t node_device(const NodeView& v, int* device) {
    if (v.device >= 0) {
        *device = v.device;
        return hipSuccess;
    }
    return hipGetDevice(device);
}

float scale_log2_for(size_t head_dim) {
    return (float)(1.4426950408889634 / std::sqrt((double)head_dim));
}

}  // namespace

long get_option(int which) {
    if (which < 0 || which >= kOptCount) return 0;
    return g_options[which].load(std::memory_order_relaxed);
}

int device_cu_count(int device) {
    if (device < 0 || device >= kMaxDevices) return 256;
    int v = g_cu_count[device].load(std::memory_order_relaxed);
    if (v > 0) return v;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        cus <= 0)
        cus = 256;
    g_cu_count[device].store(cus, std::memory_order_relaxed);
    return cus;
}

}  // namespace attn

using namespace attn;

extern "C" {

const char* attn_version(void) { return "attn_mi355x 0.1 gfx950"; }

int attn_set_option(const char* name, long value) {
    if (!name) return -1;
    int which = -1;
    if (!std::strcmp(name, "decode_force_generic")) which = kOptDecodeForceGeneric;
    else if (!std::strcmp(name, "decode_splits")) which = kOptDecodeSplits;
    else if (!std::strcmp(name, "prefill_force_generic")) which = kOptPrefillForceGeneric;
    else if (!std::strcmp(name, "decode_heads_per_workgroup")) which = kOptDecodeHeadsPerGroup;
    else if (!std::strcmp(name, "decode_kdma")) which = kOptDecodeKdma;
    else if (!std::strcmp(name, "graph_node_records")) which = kOptGraphNodeRecords;
    else if (!std::strcmp(name, "decode_whole_max_keys")) which = kOptDecodeWholeMaxKeys;
    else if (!std::strcmp(name, "qkv_gemm_force_generic")) which = kOptQkvGemmForceGeneric;
    else if (!std::strcmp(name, "qkv_gemm_tokens_per_wave")) which = kOptQkvGemmTokensPerWave;
    else if (!std::strcmp(name, "qkv_gemm_wide")) which = kOptQkvGemmWide;
    else if (!std::strcmp(name, "prefill_waves")) which = kOptPrefillWaves;
    else if (!std::strcmp(name, "decode_out_proj_fused")) which = kOptDecodeOutProjFused;
    else if (!std::strcmp(name, "prefill_stage_all")) which = kOptPrefillStageAll;
    else if (!std::strcmp(name, "prefill_split_keys")) which = kOptPrefillSplitKeys;
    else if (!std::strcmp(name, "prefill_key_halves")) which = kOptPrefillKeyHalves;
    if (which < 0) return -1;
    g_options[which].store(value, std::memory_order_relaxed);
    return 0;
}

size_t attn_graph_node_records(void) {
    NodeStore& s = node_store();
    std::lock_guard<std::mutex> lock(s.mu);
    return s.nodes.size();
}

size_t attn_decode_workspace_states(size_t num_heads, size_t kv_len) {
    return num_heads * ((kv_len + ATTN_KV_CHUNK - 1) / ATTN_KV_CHUNK);
}

int attn_rope_tables(attn_f16_t* cos_out, attn_f16_t* sin_out, size_t max_seq_len,
                     size_t head_dim, float rope_theta) {
    if (!cos_out || !sin_out || head_dim < 2) return (int)hipErrorInvalidValue;
    const size_t half = head_dim / 2;
    for (size_t i = 0; i < half; ++i) {
        const float exponent = (float)(2 * i) / (float)head_dim;
        const float inv_freq = 1.0f / std::pow(rope_theta, exponent);
        for (size_t pos = 0; pos < max_seq_len; ++pos) {
            const float angle = (float)pos * inv_freq;
            const _Float16 c = (_Float16)std::cos(angle);
            const _Float16 s = (_Float16)std::sin(angle);
            std::memcpy(&cos_out[pos * half + i], &c, 2);
            std::memcpy(&sin_out[pos * half + i], &s, 2);
        }
    }
    return 0;
}

int attn_rope_store_kv(attn_f16_t* q, attn_f16_t* k, const attn_f16_t* v,
                       attn_f16_t* k_cache, attn_f16_t* v_cache,
                       const attn_f16_t* cos_table, const attn_f16_t* sin_table,
                       size_t seq_len, size_t num_heads, size_t num_kv_heads, size_t head_dim,
                       size_t q_stride, size_t k_stride, size_t start_pos,
                       int apply_rotation, hipStream_t stream) {
    if (seq_len == 0) return 0;  // rope.hip.cpp:156
    if (head_dim == 0 || (head_dim & 1u)) return (int)hipErrorInvalidValue;
    if (!apply_rotation && k_cache == nullptr) return (int)hipErrorInvalidValue;
    if (k_cache && (!v_cache || !v)) return (int)hipErrorInvalidValue;
    if (!fits_u32(seq_len) || !fits_u32(num_heads) || !fits_u32(num_kv_heads) ||
        !fits_u32(head_dim) || !fits_u32(start_pos + seq_len))
        return (int)hipErrorInvalidValue;
    RopeArgs a{};
    a.q = reinterpret_cast<f16*>(q);
    a.k = reinterpret_cast<f16*>(k);
    a.v = reinterpret_cast<const f16*>(v);
    a.kc = reinterpret_cast<f16*>(k_cache);
    a.vc = reinterpret_cast<f16*>(v_cache);
    a.cos_t = reinterpret_cast<const f16*>(cos_table);
    a.sin_t = reinterpret_cast<const f16*>(sin_table);
    a.q_stride = q_stride ? q_stride : num_heads * head_dim;
    a.k_stride = k_stride ? k_stride : num_kv_heads * head_dim;
    a.seq_len = (uint32_t)seq_len;
    a.num_heads = (uint32_t)num_heads;
    a.num_kv_heads = (uint32_t)num_kv_heads;
    a.head_dim = (uint32_t)head_dim;
    a.start_pos = (uint32_t)start_pos;
    a.apply = apply_rotation ? 1u : 0u;
    a.lanes_per_head = (uint32_t)(head_dim / 16);
    const bool vec = rope_vector_ok(a);
    const hipError_t e = launch_rope_kernel(a, vec, stream);
    if (e == hipSuccess) remember_launch<RopeArgs>(stream);
    return (int)e;
}

int attn_rope(attn_f16_t* q, attn_f16_t* k, const attn_f16_t* cos_table,
              const attn_f16_t* sin_table, size_t seq_len, size_t num_heads,
              size_t num_kv_heads, size_t head_dim, size_t q_stride, size_t k_stride,
              size_t start_pos, hipStream_t stream) {
    return attn_rope_store_kv(q, k, nullptr, nullptr, nullptr, cos_table, sin_table, seq_len,
                              num_heads, num_kv_heads, head_dim, q_stride, k_stride, start_pos,
                              1, stream);
}

int attn_update_rope_node(hipGraphExec_t graph_exec, hipGraphNode_t node, size_t start_pos,
                          int apply_rotation) {
    NodeView view;
    hipError_t e = view_node(node, view);
    if (e != hipSuccess) return (int)e;
    hipKernelNodeParams& params = view.params;
    if (params.func != rope_kernel_symbol(true) && params.func != rope_kernel_symbol(false))
        return (int)hipErrorInvalidValue;
    RopeArgs a = *reinterpret_cast<const RopeArgs*>(view.arg);
    if (!fits_u32(start_pos + a.seq_len)) return (int)hipErrorInvalidValue;
    if (!apply_rotation && a.kc == nullptr) return (int)hipErrorInvalidValue;
    a.start_pos = (uint32_t)start_pos;
    a.apply = apply_rotation ? 1u : 0u;
    void* args[1] = {&a};
    params.kernelParams = args;
    params.extra = nullptr;
    return (int)hipGraphExecKernelNodeSetParams(graph_exec, node, &params);
}

// x and W may be null only for an empty reduction (hidden 0: y = 0).
static bool qkv_args_ok(const attn_f16_t* x, const attn_f16_t* y, const attn_f16_t* w,
                        size_t hidden, size_t out_dim) {
    return y && (hidden == 0 || (x && w)) && fits_u32(out_dim) && fits_u32(hidden) &&
           fits_u32(out_dim + 1);
}

int attn_qkv_decode(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w, size_t hidden_size,
                    size_t total_qkv_dim, hipStream_t stream) {
    if (total_qkv_dim == 0) return 0;  // matrix_vec_mul.hip.cpp:160
    if (!qkv_args_ok(x, y, w, hidden_size, total_qkv_dim)) return (int)hipErrorInvalidValue;
    QkvArgs a{};
    a.x = reinterpret_cast<const f16*>(x);
    a.w = reinterpret_cast<const f16*>(w);
    a.y = reinterpret_cast<f16*>(y);
    a.out_dim = (uint32_t)total_qkv_dim;
    a.in_dim = (uint32_t)hidden_size;
    return (int)launch_qkv_kernel(a, false, stream);
}

int attn_qkv_rope_store_kv_decode(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w,
                                  attn_f16_t* k_cache, attn_f16_t* v_cache,
                                  const attn_f16_t* cos_table, const attn_f16_t* sin_table,
                                  size_t hidden_size, size_t num_heads, size_t num_kv_heads,
                                  size_t head_dim, size_t start_pos, int apply_rotation,
                                  hipStream_t stream) {
    const size_t out_dim = (num_heads + 2 * num_kv_heads) * head_dim;
    if (out_dim == 0) return 0;
    if (!qkv_args_ok(x, y, w, hidden_size, out_dim)) return (int)hipErrorInvalidValue;
    if (head_dim & 1u || !k_cache || !v_cache || !cos_table || !sin_table || !fits_u32(start_pos))
        return (int)hipErrorInvalidValue;
    QkvArgs a{};
    a.x = reinterpret_cast<const f16*>(x);
    a.w = reinterpret_cast<const f16*>(w);
    a.y = reinterpret_cast<f16*>(y);
    a.kc = reinterpret_cast<f16*>(k_cache);
    a.vc = reinterpret_cast<f16*>(v_cache);
    a.cos_t = reinterpret_cast<const f16*>(cos_table);
    a.sin_t = reinterpret_cast<const f16*>(sin_table);
    a.out_dim = (uint32_t)out_dim;
    a.in_dim = (uint32_t)hidden_size;
    a.num_heads = (uint32_t)num_heads;
    a.num_kv_heads = (uint32_t)num_kv_heads;
    a.head_dim = (uint32_t)head_dim;
    a.start_pos = (uint32_t)start_pos;
    a.apply = apply_rotation ? 1u : 0u;
    const hipError_t e = launch_qkv_kernel(a, true, stream);
    if (e == hipSuccess) remember_launch<QkvArgs>(stream);
    return (int)e;
}

int attn_update_qkv_rope_node(hipGraphExec_t graph_exec, hipGraphNode_t node, size_t start_pos,
                              int apply_rotation) {
    NodeView view;
    hipError_t e = view_node(node, view);
    if (e != hipSuccess) return (int)e;
    hipKernelNodeParams& params = view.params;
    if (params.func != qkv_kernel_symbol(true, true) && params.func != qkv_kernel_symbol(true, false))
        return (int)hipErrorInvalidValue;
    if (!fits_u32(start_pos)) return (int)hipErrorInvalidValue;
    QkvArgs a = *reinterpret_cast<const QkvArgs*>(view.arg);
    a.start_pos = (uint32_t)start_pos;
    a.apply = apply_rotation ? 1u : 0u;
    void* args[1] = {&a};
    params.kernelParams = args;
    params.extra = nullptr;
    return (int)hipGraphExecKernelNodeSetParams(graph_exec, node, &params);
}

int attn_out_proj_decode(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w,
                         size_t hidden_size, size_t num_heads, size_t head_dim, float beta,
                         hipStream_t stream) {
    if (hidden_size == 0) return 0;  // matrix_vec_mul.hip.cpp:160
    const size_t in_dim = num_heads * head_dim;
    if (!qkv_args_ok(x, y, w, in_dim, hidden_size)) return (int)hipErrorInvalidValue;
    QkvArgs a{};
    a.x = reinterpret_cast<const f16*>(x);
    a.w = reinterpret_cast<const f16*>(w);
    a.y = reinterpret_cast<f16*>(y);
    a.out_dim = (uint32_t)hidden_size;
    a.in_dim = (uint32_t)in_dim;
    a.beta = beta;
    return (int)launch_qkv_kernel(a, false, stream);
}

static int qkv_gemm_args(QkvGemmArgs& a, const attn_f16_t* x, attn_f16_t* y,
                         const attn_f16_t* w, size_t seq_len, size_t hidden, size_t total) {
    if (!y || (hidden != 0 && (!x || !w))) return (int)hipErrorInvalidValue;
    if (!fits_u32(seq_len) || !fits_u32(hidden) || !fits_u32(total + 255))
        return (int)hipErrorInvalidValue;
    a = QkvGemmArgs{};
    a.x = reinterpret_cast<const f16*>(x);
    a.w = reinterpret_cast<const f16*>(w);
    a.y = reinterpret_cast<f16*>(y);
    a.M = (uint32_t)seq_len;
    a.N = (uint32_t)total;
    a.K = (uint32_t)hidden;
    return 0;
}

int attn_qkv_gemm(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w, size_t seq_len,
                  size_t hidden_size, size_t total_qkv_dim, hipStream_t stream) {
    if (seq_len == 0 || total_qkv_dim == 0) return 0;
    QkvGemmArgs a;
    if (int rc = qkv_gemm_args(a, x, y, w, seq_len, hidden_size, total_qkv_dim)) return rc;
    return (int)launch_qkv_gemm_kernel(a, false, stream);
}

int attn_qkv_gemm_rope_store_kv(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w,
                                attn_f16_t* k_cache, attn_f16_t* v_cache,
                                const attn_f16_t* cos_table, const attn_f16_t* sin_table,
                                size_t seq_len, size_t hidden_size, size_t num_heads,
                                size_t num_kv_heads, size_t head_dim, size_t start_pos,
                                int apply_rotation, hipStream_t stream) {
    if (seq_len == 0) return 0;
    const size_t q_dim = num_heads * head_dim, kv_dim = num_kv_heads * head_dim;
    const size_t total = q_dim + 2 * kv_dim;
    if (total == 0) return 0;
    if (head_dim & 1u || !k_cache || !v_cache || !cos_table || !sin_table ||
        !fits_u32(start_pos + seq_len))
        return (int)hipErrorInvalidValue;
    QkvGemmArgs a;
    if (int rc = qkv_gemm_args(a, x, y, w, seq_len, hidden_size, total)) return rc;
    const auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    if (head_dim == 128 && qkv_gemm_mfma_ok(a) && a16(y) && a16(k_cache) && a16(v_cache) &&
        a16(cos_table) && a16(sin_table)) {
        a.kc = reinterpret_cast<f16*>(k_cache);
        a.vc = reinterpret_cast<f16*>(v_cache);
        a.cos_t = reinterpret_cast<const f16*>(cos_table);
        a.sin_t = reinterpret_cast<const f16*>(sin_table);
        a.num_heads = (uint32_t)num_heads;
        a.num_kv_heads = (uint32_t)num_kv_heads;
        a.start_pos = (uint32_t)start_pos;
        a.apply = apply_rotation ? 1u : 0u;
        return (int)launch_qkv_gemm_kernel(a, true, stream);
    }
    // other shapes: the two launches the fused kernel replaces
    if (hipError_t e = launch_qkv_gemm_kernel(a, false, stream)) return (int)e;
    return attn_rope_store_kv(y, y + q_dim, y + q_dim + kv_dim, k_cache, v_cache, cos_table,
                              sin_table, seq_len, num_heads, num_kv_heads, head_dim, total, total,
                              start_pos, apply_rotation, stream);
}

int attn_prefill_plan(const void* q, const void* k, const void* v, const void* out,
                      size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t q_stride,
                      size_t kv_stride) {
    if (num_kv_heads == 0 || num_heads % num_kv_heads != 0) return -1;
    PrefillArgs a{};
    a.q = reinterpret_cast<const f16*>(q);
    a.k = reinterpret_cast<const f16*>(k);
    a.v = reinterpret_cast<const f16*>(v);
    a.out = reinterpret_cast<f16*>(const_cast<void*>(out));
    a.q_stride = q_stride ? q_stride : num_heads * head_dim;
    a.kv_stride = kv_stride ? kv_stride : num_kv_heads * head_dim;
    a.num_heads = (uint32_t)num_heads;
    a.num_kv_heads = (uint32_t)num_kv_heads;
    a.group = (uint32_t)(num_heads / num_kv_heads);
    a.head_dim = (uint32_t)head_dim;
    return plan_prefill(a);
}

int attn_prefill(const attn_f16_t* q, const attn_f16_t* k, const attn_f16_t* v,
                 attn_f16_t* out, size_t seq_len, size_t num_heads, size_t num_kv_heads,
                 size_t head_dim, size_t q_stride, size_t kv_stride, hipStream_t stream) {
    // causal_attention.hip.cpp:392-399
    if (seq_len == 0 || num_kv_heads == 0) return 0;
    if (num_heads % num_kv_heads != 0) return 0;
    if (head_dim == 0) return 0;
    if (!fits_u32(seq_len) || !fits_u32(num_heads) || !fits_u32(head_dim))
        return (int)hipErrorInvalidValue;
    if (!q || !k || !v || !out) return (int)hipErrorInvalidValue;
    PrefillArgs a{};
    a.q = reinterpret_cast<const f16*>(q);
    a.k = reinterpret_cast<const f16*>(k);
    a.v = reinterpret_cast<const f16*>(v);
    a.out = reinterpret_cast<f16*>(out);
    a.q_stride = q_stride ? q_stride : num_heads * head_dim;
    a.kv_stride = kv_stride ? kv_stride : num_kv_heads * head_dim;
    a.seq_len = (uint32_t)seq_len;
    a.num_heads = (uint32_t)num_heads;
    a.num_kv_heads = (uint32_t)num_kv_heads;
    a.group = (uint32_t)(num_heads / num_kv_heads);
    a.head_dim = (uint32_t)head_dim;
    a.q_tiles = (uint32_t)((seq_len + 63) / 64);
    a.scale_log2 = scale_log2_for(head_dim);
    const int path = plan_prefill(a);
    if (path == 1) return (int)launch_prefill_kernel(a, path, stream);
    GenericAttnArgs g{};
    g.q = a.q;
    g.k = a.k;
    g.v = a.v;
    g.out = a.out;
    g.q_stride = a.q_stride;
    g.kv_stride = a.kv_stride;
    g.nq = a.seq_len;
    g.kv_len = a.seq_len;
    g.num_heads = a.num_heads;
    g.group = a.group;
    g.head_dim = a.head_dim;
    g.causal = 1;
    g.scale_log2 = a.scale_log2;
    return (int)launch_generic_attention(g, stream);
}

int attn_decode_plan(size_t kv_len, size_t num_heads, size_t num_kv_heads, size_t head_dim,
                     size_t kv_stride, const void* q, const void* k_cache,
                     const void* v_cache, uint32_t out[5]) {
    if (!out || num_kv_heads == 0 || num_heads % num_kv_heads != 0 || kv_len == 0) return -1;
    int device = 0;
    (void)hipGetDevice(&device);
    const size_t kvs = kv_stride ? kv_stride : num_kv_heads * head_dim;
    const DecodePlan p = plan_decode((uint32_t)kv_len, (uint32_t)num_heads,
                                     (uint32_t)num_kv_heads, (uint32_t)head_dim, kvs, q,
                                     k_cache, v_cache, device, true);
    out[0] = (uint32_t)p.path;
    out[1] = p.nsplit;
    out[2] = p.chunk;
    out[3] = p.block;
    out[4] = p.nstate;
    return 0;
}

// Enqueue an MFMA decode plan as the reference does: the split kernel
// (*attention_node) then the merge kernel (*merge_node).  A whole-context
// plan is the split kernel alone, unless the caller asks for the merge node
// (a graph whose updaters may move to a longer context): then the merge
// kernel is enqueued too and exits at once while the plan stays whole.
static int enqueue_decode(DecodeArgs& a, int device, bool rope, hipStream_t stream,
                          hipGraphNode_t* attention_node, hipGraphNode_t* merge_node) {
    a.whole_ok = 1;
    const DecodePlan p = replan_decode(a, device);
    if (p.path < 1 || p.path > 3) return (int)hipErrorInvalidValue;
    hipError_t e = launch_decode_split(a, p, stream, rope);
    if (e != hipSuccess) return (int)e;
    remember_launch<DecodeArgs>(stream);
    if (attention_node) {
        e = captured_node(stream, attention_node);
        if (e != hipSuccess) return (int)e;
    }
    if (p.whole && !merge_node) return 0;
    e = launch_decode_merge(a, stream, rope);
    if (e != hipSuccess) return (int)e;
    remember_launch<DecodeArgs>(stream);
    if (merge_node) {
        e = captured_node(stream, merge_node);
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

int attn_decode(const attn_f16_t* q, const attn_f16_t* k_cache, const attn_f16_t* v_cache,
                attn_f16_t* out, float* partial_out, float* partial_max, float* partial_sum,
                size_t query_len, size_t kv_len, size_t start_pos, size_t num_heads,
                size_t num_kv_heads, size_t head_dim, size_t q_stride, size_t kv_stride,
                hipStream_t stream, hipGraphNode_t* attention_node, hipGraphNode_t* merge_node) {
    (void)start_pos;  // all kv_len keys are visible (causal_attention.hip.cpp:943)
    (void)q_stride;   // q is read packed [num_heads][head_dim] (:944)
    // causal_attention.hip.cpp:860-866, :945-946
    if (query_len == 0 || kv_len == 0 || num_kv_heads == 0 || head_dim == 0) return 0;
    if (num_heads % num_kv_heads != 0) return 0;
    if (!fits_u32(kv_len) || !fits_u32(num_heads) || !fits_u32(head_dim))
        return (int)hipErrorInvalidValue;
    if (!q || !k_cache || !v_cache || !out) return (int)hipErrorInvalidValue;
    const size_t kvs = kv_stride ? kv_stride : num_kv_heads * head_dim;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return (int)e;
    const DecodePlan p = plan_decode((uint32_t)kv_len, (uint32_t)num_heads,
                                     (uint32_t)num_kv_heads, (uint32_t)head_dim, kvs, q,
                                     k_cache, v_cache, device, true);
    if (p.path == 0) {
        // one kernel: both node handles name it (the merge patcher is a no-op)
        GenericAttnArgs g{};
        g.q = reinterpret_cast<const f16*>(q);
        g.k = reinterpret_cast<const f16*>(k_cache);
        g.v = reinterpret_cast<const f16*>(v_cache);
        g.out = reinterpret_cast<f16*>(out);
        g.q_stride = num_heads * head_dim;
        g.kv_stride = kvs;
        g.nq = 1;
        g.kv_len = (uint32_t)kv_len;
        g.num_heads = (uint32_t)num_heads;
        g.group = (uint32_t)(num_heads / num_kv_heads);
        g.head_dim = (uint32_t)head_dim;
        g.causal = 0;
        g.scale_log2 = scale_log2_for(head_dim);
        e = launch_generic_attention(g, stream);
        if (e != hipSuccess) return (int)e;
        remember_launch<GenericAttnArgs>(stream);
        if (attention_node || merge_node) {
            hipGraphNode_t node = nullptr;
            e = captured_node(stream, &node);
            if (e != hipSuccess) return (int)e;
            if (attention_node) *attention_node = node;
            if (merge_node) *merge_node = node;
        }
        return 0;
    }
    if (!partial_out || !partial_max || !partial_sum) return (int)hipErrorInvalidValue;
    DecodeArgs a{};
    a.q = reinterpret_cast<const f16*>(q);
    a.k = reinterpret_cast<const f16*>(k_cache);
    a.v = reinterpret_cast<const f16*>(v_cache);
    a.out = reinterpret_cast<f16*>(out);
    a.part_out = partial_out;
    a.part_max = partial_max;
    a.part_sum = partial_sum;
    a.kv_stride = kvs;
    a.kv_len = (uint32_t)kv_len;
    a.num_heads = (uint32_t)num_heads;
    a.num_kv_heads = (uint32_t)num_kv_heads;
    a.group = (uint32_t)(num_heads / num_kv_heads);
    a.head_dim = (uint32_t)head_dim;
    a.scale_log2 = scale_log2_for(head_dim);
    return enqueue_decode(a, device, false, stream, attention_node, merge_node);
}

int attn_rope_store_kv_decode(attn_f16_t* q, const attn_f16_t* k, const attn_f16_t* v,
                              attn_f16_t* k_cache, attn_f16_t* v_cache,
                              const attn_f16_t* cos_table, const attn_f16_t* sin_table,
                              attn_f16_t* out, float* partial_out, float* partial_max,
                              float* partial_sum, size_t kv_len, size_t start_pos,
                              size_t num_heads, size_t num_kv_heads, size_t head_dim,
                              size_t kv_stride, int apply_rotation, hipStream_t stream,
                              hipGraphNode_t* attention_node, hipGraphNode_t* merge_node) {
    // the no-op shapes of both replaced launches (rope.hip.cpp:156,
    // causal_attention.hip.cpp:860-866, :945-946)
    if (kv_len == 0 || num_kv_heads == 0 || head_dim == 0) return 0;
    if (num_heads % num_kv_heads != 0) return 0;
    if (!fits_u32(kv_len) || !fits_u32(num_heads) || !fits_u32(head_dim))
        return (int)hipErrorInvalidValue;
    if (!q || !k || !v || !k_cache || !v_cache || !out || !partial_out || !partial_max ||
        !partial_sum)
        return (int)hipErrorInvalidValue;
    if (apply_rotation && (!cos_table || !sin_table)) return (int)hipErrorInvalidValue;
    const size_t kv_dim = num_kv_heads * head_dim;
    const size_t kvs = kv_stride ? kv_stride : kv_dim;
    // the fused kernels serve the MFMA decode path with the engine's cache
    // layout (RoPE writes rows kv_dim apart, rope.hip.cpp:110) and the new
    // token inside the decoded range
    const bool al = ((uintptr_t)k | (uintptr_t)v | (uintptr_t)cos_table | (uintptr_t)sin_table |
                     (uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0;
    const bool host_ok = al && kvs == kv_dim && start_pos < kv_len;
    // Other shapes: eager calls issue the two launches this replaces; a
    // capture asking for node handles is rejected (hipErrorInvalidValue,
    // nothing enqueued), because attn_update_rope_decode_nodes could not
    // patch that sequence as one pair
    if (!host_ok && (attention_node || merge_node)) return (int)hipErrorInvalidValue;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return (int)e;
    const DecodePlan p = plan_decode((uint32_t)kv_len, (uint32_t)num_heads,
                                     (uint32_t)num_kv_heads, (uint32_t)head_dim, kvs, q,
                                     k_cache, v_cache, device, true);
    if (p.path == 0 || !host_ok) {
        if (attention_node || merge_node) return (int)hipErrorInvalidValue;
        const int rc = attn_rope_store_kv(q, const_cast<attn_f16_t*>(k), v, k_cache, v_cache,
                                          cos_table, sin_table, 1, num_heads, num_kv_heads,
                                          head_dim, 0, 0, start_pos, apply_rotation, stream);
        if (rc != 0) return rc;
        return attn_decode(q, k_cache, v_cache, out, partial_out, partial_max, partial_sum, 1,
                           kv_len, start_pos, num_heads, num_kv_heads, head_dim, 0, kv_stride,
                           stream, nullptr, nullptr);
    }
    DecodeArgs a{};
    a.q = reinterpret_cast<const f16*>(q);
    a.k = reinterpret_cast<const f16*>(k_cache);
    a.v = reinterpret_cast<const f16*>(v_cache);
    a.out = reinterpret_cast<f16*>(out);
    a.part_out = partial_out;
    a.part_max = partial_max;
    a.part_sum = partial_sum;
    a.kv_stride = kvs;
    a.kv_len = (uint32_t)kv_len;
    a.num_heads = (uint32_t)num_heads;
    a.num_kv_heads = (uint32_t)num_kv_heads;
    a.group = (uint32_t)(num_heads / num_kv_heads);
    a.head_dim = (uint32_t)head_dim;
    a.scale_log2 = scale_log2_for(head_dim);
    a.q_rot = reinterpret_cast<f16*>(q);
    a.k_dst = reinterpret_cast<f16*>(k_cache);
    a.v_dst = reinterpret_cast<f16*>(v_cache);
    a.k_src = reinterpret_cast<const f16*>(k);
    a.v_src = reinterpret_cast<const f16*>(v);
    a.cos_t = reinterpret_cast<const f16*>(cos_table);
    a.sin_t = reinterpret_cast<const f16*>(sin_table);
    a.row = (uint32_t)start_pos;
    a.apply = apply_rotation ? 1u : 0u;
    return enqueue_decode(a, device, true, stream, attention_node, merge_node);
}

size_t attn_decode_out_proj_workspace_bytes(size_t num_heads, size_t hidden_size) {
    return out_proj_workspace_bytes(num_heads, hidden_size);
}

int attn_decode_out_proj(const attn_f16_t* q, const attn_f16_t* k_cache, const attn_f16_t* v_cache,
                         attn_f16_t* attn_out, float* partial_out, float* partial_max,
                         float* partial_sum, size_t kv_len, size_t num_heads,
                         size_t num_kv_heads, size_t head_dim, size_t kv_stride,
                         const attn_f16_t* w_o, attn_f16_t* y, size_t hidden_size, float beta,
                         void* out_proj_workspace, hipStream_t stream,
                         hipGraphNode_t* attention_node, hipGraphNode_t* merge_node) {
    // the two launches this replaces, in the engine's order
    // (model_inference.hpp:371-397), for every shape the fused kernel does
    // not serve (their own no-op and error rules apply)
    const auto two_launches = [&]() -> int {
        int rc = attn_decode(q, k_cache, v_cache, attn_out, partial_out, partial_max,
                             partial_sum, 1, kv_len, kv_len ? kv_len - 1 : 0, num_heads,
                             num_kv_heads, head_dim, 0, kv_stride, stream, attention_node,
                             merge_node);
        if (rc != 0) return rc;
        return attn_out_proj_decode(attn_out, y, w_o, hidden_size, num_heads, head_dim, beta,
                                    stream);
    };
    // the two launches unless the fused kernel is asked for: on MI355X it is
    // the slower form (its cross-XCD reduction of the heads costs more than
    // the kernel boundary it removes)
    if (get_option(kOptDecodeOutProjFused) != 1 || hidden_size == 0 || kv_len == 0 ||
        num_kv_heads == 0 || head_dim == 0 || num_heads % num_kv_heads != 0 ||
        !out_proj_workspace || !w_o || !y)
        return two_launches();
    if (!fits_u32(kv_len) || !fits_u32(num_heads) || !fits_u32(head_dim) ||
        !fits_u32(hidden_size))
        return (int)hipErrorInvalidValue;
    if (!q || !k_cache || !v_cache || !attn_out || !partial_out || !partial_max || !partial_sum)
        return (int)hipErrorInvalidValue;
    const size_t kvs = kv_stride ? kv_stride : num_kv_heads * head_dim;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return (int)e;
    OutProjArgs o{};
    DecodeArgs& a = o.d;
    a.q = reinterpret_cast<const f16*>(q);
    a.k = reinterpret_cast<const f16*>(k_cache);
    a.v = reinterpret_cast<const f16*>(v_cache);
    a.out = reinterpret_cast<f16*>(attn_out);
    a.part_out = partial_out;
    a.part_max = partial_max;
    a.part_sum = partial_sum;
    a.kv_stride = kvs;
    a.kv_len = (uint32_t)kv_len;
    a.num_heads = (uint32_t)num_heads;
    a.num_kv_heads = (uint32_t)num_kv_heads;
    a.group = (uint32_t)(num_heads / num_kv_heads);
    a.head_dim = (uint32_t)head_dim;
    a.scale_log2 = scale_log2_for(head_dim);
    o.w = reinterpret_cast<const f16*>(w_o);
    o.y = reinterpret_cast<f16*>(y);
    o.hidden = (uint32_t)hidden_size;
    o.row_blocks = (uint32_t)((hidden_size + kOutProjRows - 1) / kOutProjRows);
    o.beta = beta;
    o.xcd_map = num_heads % 8 == 0 ? 1u : 0u;
    const size_t part = out_proj_workspace_bytes(num_heads, hidden_size) -
                        (size_t)o.row_blocks * sizeof(uint32_t);
    o.y_part = static_cast<float*>(out_proj_workspace);
    o.counters = reinterpret_cast<uint32_t*>(static_cast<char*>(out_proj_workspace) + part);
    // whole_ok = 0: the fused form always splits, so that its merge node stays
    // a merge at every context an updater moves it to
    const DecodePlan p = replan_decode(a, device);
    if (p.path < 1 || p.path > 3 || !out_proj_fused_ok(o)) return two_launches();
    e = launch_decode_split(a, p, stream, false);
    if (e != hipSuccess) return (int)e;
    remember_launch<DecodeArgs>(stream);
    if (attention_node) {
        e = captured_node(stream, attention_node);
        if (e != hipSuccess) return (int)e;
    }
    e = launch_merge_out_proj(o, stream, false);
    if (e != hipSuccess) return (int)e;
    remember_launch<OutProjArgs>(stream);
    if (merge_node) {
        e = captured_node(stream, merge_node);
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

// Re-point a captured split node at kv_len: its kernel (heads per
// workgroup), grid and arguments.
static hipError_t replan_split_node(hipGraphExec_t graph_exec, hipGraphNode_t node,
                                    hipKernelNodeParams& params, DecodeArgs& a, bool rope,
                                    int device) {
    const DecodePlan p = replan_decode(a, device);
    if (p.path < 1 || p.path > 3) return hipErrorInvalidValue;
    void* args[1] = {&a};
    params.kernelParams = args;
    params.extra = nullptr;
    params.func = const_cast<void*>(decode_split_symbol(p, rope));
    params.gridDim = decode_grid(a, p);
    return hipGraphExecKernelNodeSetParams(graph_exec, node, &params);
}

// Re-point a captured merge node at kv_len (its split count; for a
// whole-context plan the idle kernel).
static hipError_t replan_merge_node(hipGraphExec_t graph_exec, hipGraphNode_t node,
                                    hipKernelNodeParams& params, DecodeArgs& a, bool rope,
                                    int device) {
    const DecodePlan p = replan_decode(a, device);
    if (p.path < 1 || p.path > 3) return hipErrorInvalidValue;
    void* args[1] = {&a};
    params.kernelParams = args;
    params.extra = nullptr;
    params.func = const_cast<void*>(decode_merge_symbol(rope, a.whole != 0));
    params.gridDim = decode_merge_grid(a);
    return hipGraphExecKernelNodeSetParams(graph_exec, node, &params);
}

int attn_update_rope_decode_nodes(hipGraphExec_t graph_exec, hipGraphNode_t attention_node,
                                  hipGraphNode_t merge_node, size_t kv_len, size_t start_pos,
                                  int apply_rotation) {
    if (kv_len == 0 || !fits_u32(kv_len) || start_pos >= kv_len) return (int)hipErrorInvalidValue;
    for (int m = 0; m < 2; ++m) {
        hipGraphNode_t node = m ? merge_node : attention_node;
        NodeView view;
        hipError_t e = view_node(node, view);
        if (e != hipSuccess) return (int)e;
        int device = 0;
        e = node_device(view, &device);
        if (e != hipSuccess) return (int)e;
        hipKernelNodeParams& params = view.params;
        const bool ok = m ? (params.func == decode_merge_symbol(true, false) ||
                             params.func == decode_merge_symbol(true, true))
                          : decode_path_of_symbol(params.func, true) != 0;
        if (!ok) return (int)hipErrorInvalidValue;
        DecodeArgs a = *reinterpret_cast<const DecodeArgs*>(view.arg);
        const uint64_t captured = merge_sig(a);
        a.kv_len = (uint32_t)kv_len;
        a.row = (uint32_t)start_pos;
        a.apply = apply_rotation ? 1u : 0u;
        if (a.apply && (!a.cos_t || !a.sin_t)) return (int)hipErrorInvalidValue;
        if (!m) {
            e = replan_split_node(graph_exec, node, params, a, true, device);
            if (e != hipSuccess) return (int)e;
            continue;
        }
        const DecodePlan p = replan_decode(a, device);
        if (p.path < 1 || p.path > 3) return (int)hipErrorInvalidValue;
        if (merge_current(graph_exec, node, captured, merge_sig(a))) continue;
        e = replan_merge_node(graph_exec, node, params, a, true, device);
        if (e != hipSuccess) return (int)e;
        merge_patched(graph_exec, node, merge_sig(a));
    }
    return 0;
}

static int patch_decode_node(hipGraphExec_t graph_exec, hipGraphNode_t node, size_t kv_len,
                             bool merge) {
    if (kv_len == 0 || !fits_u32(kv_len)) return (int)hipErrorInvalidValue;
    NodeView view;
    hipError_t e = view_node(node, view);
    if (e != hipSuccess) return (int)e;
    hipKernelNodeParams& params = view.params;
    if (params.func == generic_attention_symbol()) {
        if (merge) return 0;  // single-kernel path: nothing separate to patch
        GenericAttnArgs g = *reinterpret_cast<const GenericAttnArgs*>(view.arg);
        if (g.causal) return (int)hipErrorInvalidValue;  // a prefill node, not decode
        g.kv_len = (uint32_t)kv_len;
        void* args[1] = {&g};
        params.kernelParams = args;
        params.extra = nullptr;
        return (int)hipGraphExecKernelNodeSetParams(graph_exec, node, &params);
    }
    int device = 0;
    if (params.func == merge_out_proj_symbol(false)) {
        // the merge fused into o_proj: its decode arguments follow kv_len
        if (!merge) return (int)hipErrorInvalidValue;
        OutProjArgs o = *reinterpret_cast<const OutProjArgs*>(view.arg);
        e = node_device(view, &device);
        if (e != hipSuccess) return (int)e;
        o.d.kv_len = (uint32_t)kv_len;
        const DecodePlan p = replan_decode(o.d, device);
        if (p.path < 1 || p.path > 3) return (int)hipErrorInvalidValue;
        void* args[1] = {&o};
        params.kernelParams = args;
        params.extra = nullptr;
        return (int)hipGraphExecKernelNodeSetParams(graph_exec, node, &params);
    }
    const bool is_split = decode_path_of_symbol(params.func, false) != 0;
    const bool is_merge = params.func == decode_merge_symbol(false, false) ||
                          params.func == decode_merge_symbol(false, true);
    if ((merge && !is_merge) || (!merge && !is_split)) return (int)hipErrorInvalidValue;
    DecodeArgs a = *reinterpret_cast<const DecodeArgs*>(view.arg);
    e = node_device(view, &device);
    if (e != hipSuccess) return (int)e;
    const uint64_t captured = merge_sig(a);
    a.kv_len = (uint32_t)kv_len;
    if (!merge) return (int)replan_split_node(graph_exec, node, params, a, false, device);
    const DecodePlan p = replan_decode(a, device);
    if (p.path < 1 || p.path > 3) return (int)hipErrorInvalidValue;
    // the exec node already reads this many states
    if (merge_current(graph_exec, node, captured, merge_sig(a))) return 0;
    e = replan_merge_node(graph_exec, node, params, a, false, device);
    if (e != hipSuccess) return (int)e;
    merge_patched(graph_exec, node, merge_sig(a));
    return 0;
}

int attn_update_decode_node(hipGraphExec_t graph_exec, hipGraphNode_t node, size_t kv_len) {
    return patch_decode_node(graph_exec, node, kv_len, false);
}

int attn_update_merge_node(hipGraphExec_t graph_exec, hipGraphNode_t node, size_t kv_len) {
    return patch_decode_node(graph_exec, node, kv_len, true);
}

}  // extern "C"
